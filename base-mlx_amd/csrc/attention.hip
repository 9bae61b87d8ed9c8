// GQA scaled-dot-product attention over the preallocated KV cache (gfx950).
//
// Semantics restated: mlx_rs::fast::scaled_dot_product_attention(q, k, v,
// scale, mask) as called by Qwen3::forward_internal
// (crates/base-mlx-core/src/model/qwen3.rs:491-518):
//   out = softmax(scale * q k^T + mask) v  in fp32, bf16 result;
// query head h reads kv head h / (Hq / Hkv) (GQA, qwen3.rs:491-495); with
// M > 1 new tokens the additive -1e9 mask of causal_mask_offset
// (qwen3.rs:629-653) lets query t attend keys j <= offset + t, which is
// applied here as a predicate (masked keys contribute exactly 0).
//
// Kernels chosen by the number of query rows per kv head (R = new tokens x
// q heads per kv head):
//   R <= 64 (decode, speculative verify): attn_decode_kernel splits the key
//     range over workgroups of 256 keys (flash-decoding), and the last
//     workgroup of each kv head to finish merges the unnormalised partials
//     (o, m, l);
//   otherwise (prefill): flash attention walking all visible keys,
//     attn_flash32_kernel (32 queries per wave, a GQA group per workgroup)
//     where the q heads per kv head are a power of two, else
//     attn_prefill_kernel (16 queries per wave).
// All run Q K^T and (prefill) P V on the matrix cores.
#include <math.h>

#include <algorithm>
#include <mutex>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr int kD = 128;  // head_dim

struct AttnParams {
  const uint16_t* q;  // [Hq, M, 128]; fused prologue: raw q projection rows [M, Hq*128]
  const uint16_t* k;  // [Hkv, cap, 128]
  const uint16_t* v;  // [Hkv, cap, 128]
  uint16_t* out;      // [M, Hq*128]
  float* part_o;      // [Hq, M, NS, 128]
  float* part_ml;     // [Hq, M, NS, 2]
  unsigned* cnt;      // [Hkv, row tiles] arrival counters, zero between calls
  const int* offset_dev;
  int offset;
  int Hq, Hkv, M, cap;
  int tq;     // query tokens per workgroup
  int ns;     // key splits
  int causal;
  float scale;
  int kps;    // keys per split (decode kernel: a multiple of 32, at most 256)
  int local;  // decode kernel: every workgroup of a kv head runs on one XCD (shares its L2)
};

// Inputs of the fused QK-norm + RoPE + KV-write prologue of the decode
// kernel (the operation of qk_norm_rope_kv_kernel): raw k / v projection
// rows, the q / k norm weights and the rope table.
struct FuseParams {
  const uint16_t* k_new;  // [M, Hkv*128]
  const uint16_t* v_new;  // [M, Hkv*128]
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  float eps;
  RopeTable tab;
};

// In general the split partials travel between workgroups on different XCDs
// (each with its own L2).  Every access to them is then agent-coherent: the writers store
// them with agent-scope atomic stores (relaxed, issued with sc1: written
// through to memory), every thread waits for its stores to complete
// (s_waitcnt), the workgroup meets at a barrier, and one thread bumps the
// arrival counter (a relaxed agent-scope atomic); after the next barrier
// the last arrival's threads read the partials with sc1 loads, which are
// served coherently across the L2s.  The stores have completed before the
// increment is issued and the loads are issued after it returned, so the
// loads see them; no L2 write-back (release) or invalidation (acquire) is
// needed, and these cost microseconds when many workgroups issue them.
// This holds only while store_part2<false> (and the s_waitcnt before the arrival)
// stays the only way the partials are written: a plain store into the
// split workspace could sit in one XCD's L2, and would need the release
// increment and the acquire fence back.
// Pairs of floats are stored as one 8-byte access (8-byte aligned addresses).
//
// XCD-local variant (AttnParams::local).  The hardware hands the workgroups
// of a launch to the XCDs round-robin by linear workgroup id, so with the
// kv head on the grid's x axis and a multiple of 8 kv heads, every
// workgroup of one kv head runs on the same XCD (checked on the device
// before the variant is first used: xcd_local_ok).  The partials and the
// arrival then never leave that XCD's L2: plain stores (complete once the
// L2 holds them), an increment executed in the L2 (workgroup scope), and
// merge loads with sc0, which miss in the merging CU's L1 and are served by
// the L2.  The local counters live 256 bytes from the agent-scope ones
// (kLocalCounter), so a cache line is only ever updated in one place: in
// memory by agent-scope increments or in an L2 by local ones.  Every
// launch leaves each counter at zero, and writes every partial it merges
// (on the merging XCD) before reading it, so nothing that another XCD's L2
// held from an earlier launch is read.
template <bool LOCAL>
__device__ __forceinline__ void store_part2(float* a, float x, float y) {
  if constexpr (LOCAL) {
    *reinterpret_cast<float2*>(a) = make_float2(x, y);
  } else {
    const uint64_t v =
        static_cast<uint64_t>(__float_as_uint(x)) | (static_cast<uint64_t>(__float_as_uint(y)) << 32);
    __hip_atomic_store(reinterpret_cast<uint64_t*>(a), v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Third word of a raw gfx9 buffer resource (no format conversion, range
// checked against num_records in bytes)
constexpr int kBufferConfig = 0x00020000;
// Buffer-load cache policies: sc1 (agent-coherent) and sc0 (misses in L1,
// served by the XCD's L2)
constexpr int kAgentCoherent = 16;
constexpr int kL2Coherent = 1;


typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8_t;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8_t;
typedef __attribute__((ext_vector_type(2))) _Float16 f16x2_t;
typedef __attribute__((ext_vector_type(2))) unsigned short u16x2_t;
typedef __attribute__((ext_vector_type(4))) float f32x4_t;
typedef __attribute__((ext_vector_type(2))) float f32x2_t;

// A running (max, sum, o) of softmax partials while merging splits: lane l
// holds dims 4 (l % 32) .. + 3 of the splits of parity l / 32.
struct Fold {
  float mx, l;
  float o[4];
};

// Folds the partials of splits [0, ns) of NR (head, token) rows wids[i]
// into r[i]; one wave.  Splits come in batches of 48 at fixed boundaries:
// lane s loads the (max, sum) pair of split s0 + s (one load per row), and
// each 16-byte load of o partials brings split s0 + 2u to lanes 0-31 and
// split s0 + 2u + 1 to lanes 32-63 (up to 24 loads per row and batch, one
// per pair of splits present, every load of the batch issued before the
// first is used; an odd count's last upper half reads the last split
// again, from a clamped address, and is never weighted).  The weights exp(m_s - max) come from
// the lane that holds m_s; a split without visible keys (m = -inf) is left
// out -- how many such trailing splits a launch has depends on its
// context, not on the row, so they leave a row's bits unchanged.  Each half
// of the wave folds its splits in increasing order; the halves are added at
// the end (merge_halves).
template <int NR, int AUX>
__device__ __forceinline__ void combine_splits(const AttnParams& p, const int (&wids)[NR], int lane, int ns,
                                               Fold (&r)[NR]) {
  constexpr int B = 24;  // 16-byte o loads per row and batch: 48 splits
  const int half = lane >> 5, dl = 4 * (lane & 31);
#pragma unroll
  for (int i = 0; i < NR; i++) r[i] = Fold{-INFINITY, 0.0f, {0.0f, 0.0f, 0.0f, 0.0f}};
  for (int s0 = 0; s0 < ns; s0 += 2 * B) {
    const int nb = min(2 * B, ns - s0);
    f32x2_t ml[NR];
    f32x4_t ov[NR][B];
#pragma unroll
    for (int i = 0; i < NR; i++) {
      // wids[i] is the same in every lane (it follows from the wave index);
      // reading it from lane 0 lets the buffer resources live in scalar
      // registers
      const int64_t base = static_cast<int64_t>(__builtin_amdgcn_readfirstlane(wids[i])) * p.ns + s0;
      const __amdgpu_buffer_rsrc_t rml = __builtin_amdgcn_make_buffer_rsrc(
          p.part_ml + base * 2, static_cast<short>(0), nb * 8, kBufferConfig);
      const __amdgpu_buffer_rsrc_t ro = __builtin_amdgcn_make_buffer_rsrc(
          p.part_o + base * kD, static_cast<short>(0), nb * kD * 4, kBufferConfig);
      ml[i] = __builtin_bit_cast(f32x2_t, __builtin_amdgcn_raw_buffer_load_b64(rml, min(lane, nb - 1) * 8, 0, AUX));
#pragma unroll
      for (int u = 0; u < B; u++) {
        // only the pairs that hold splits (uniform); the fold stops there
        ov[i][u] = 2 * u < nb ? __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                                                ro, (min(2 * u + half, nb - 1) * kD + dl) * 4, 0, AUX))
                              : f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      }
    }
    // every load of the batch goes out before any use of the first
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < NR; i++) {
      const float m = lane < nb ? ml[i].x : -INFINITY;
      const float bm = max_xor32(max_xor16(row16_max(m)));
      const float nm = fmaxf(r[i].mx, bm);
      if (nm == -INFINITY) continue;  // uniform: nothing visible so far
      const float a = (r[i].mx == -INFINITY) ? 0.0f : expf(r[i].mx - nm);
      const float w = (m == -INFINITY) ? 0.0f : expf(m - nm);
      // batch sum of w_s l_s: lane s holds split s; fixed butterfly order
      float wl = w * (lane < nb ? ml[i].y : 0.0f);
      wl = add_xor32(add_xor16(row16_sum(wl)));
      r[i].l = __builtin_fmaf(r[i].l, a, wl);
      r[i].mx = nm;
#pragma unroll
      for (int d = 0; d < 4; d++) r[i].o[d] *= a;
#pragma unroll
      for (int u = 0; u < B; u++) {
        if (2 * u >= nb) break;  // uniform
        const float m_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), 2 * u));
        const float m_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(m), min(2 * u + 1, 63)));
        const float w_lo = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), 2 * u));
        const float w_hi = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), min(2 * u + 1, 63)));
        const float ms = half ? m_hi : m_lo, ws = half ? w_hi : w_lo;
        if (ms != -INFINITY) {
#pragma unroll
          for (int d = 0; d < 4; d++) r[i].o[d] = __builtin_fmaf(ws, ov[i][u][d], r[i].o[d]);
        }
      }
    }
  }
}

// Normalises a merged row (the two halves of the wave added) and writes it:
// row `wid` = (head h, token t); lanes 0-31 store 4 dims each.
__device__ __forceinline__ void store_fold(const AttnParams& p, int wid, int lane, const Fold& r) {
  float o[4];
#pragma unroll
  for (int d = 0; d < 4; d++) o[d] = add_xor32(r.o[d]);
  if (lane >= 32) return;
  const int h = wid / p.M, t = wid - h * p.M;
  const float inv = r.l > 0.0f ? 1.0f / r.l : 0.0f;
  uint16_t* dst = p.out + static_cast<int64_t>(t) * p.Hq * kD + h * kD + 4 * lane;
  const uint32_t w0 = static_cast<uint32_t>(f2bf(o[0] * inv)) | (static_cast<uint32_t>(f2bf(o[1] * inv)) << 16);
  const uint32_t w1 = static_cast<uint32_t>(f2bf(o[2] * inv)) | (static_cast<uint32_t>(f2bf(o[3] * inv)) << 16);
  *reinterpret_cast<uint2*>(dst) = make_uint2(w0, w1);
}

// The merge by the last workgroup of a (kv head, row tile): rows w0 ..
// w0 + RT - 1, one per wave; with more rows than waves, a wave folds two
// rows with the loads of both in flight together.  AUX: the cache policy of
// the partial loads.
template <int NW, int AUX>
__device__ __forceinline__ void merge_rows(const AttnParams& p, int w0, int RT, int wave, int lane, int ns) {
  if (RT <= NW) {
    if (wave < RT) {
      const int wid[1] = {w0 + wave};
      Fold r[1];
      combine_splits<1, AUX>(p, wid, lane, ns, r);
      store_fold(p, wid[0], lane, r[0]);
    }
  } else {
    const int rb = min(wave + NW, RT - 1);
    const int wid[2] = {w0 + wave, w0 + rb};
    Fold r[2];
    combine_splits<2, AUX>(p, wid, lane, ns, r);
    store_fold(p, wid[0], lane, r[0]);
    if (wave + NW < RT) store_fold(p, wid[1], lane, r[1]);
  }
}


// Decode / short verify (R = tokens x heads-per-kv-head query rows of one kv
// head, up to 64).  A workgroup of NW waves owns one kv head, one tile of
// RMAX <= 8 of those rows and 32 NW keys, 32 per wave.  Every K, V and q
// load of a wave is issued before any arithmetic:
//   QK on MFMA (v_mfma_f32_16x16x32_bf16): A = the tile's query rows (padded
//     to 16; lane l holds row l%16, dims 32*ks + 8*(l/16), 4 fragments; the
//     R rows of one kv head are contiguous in [Hq, M, 128]), B = K^T (lane l
//     holds key l%16 of each 16-key tile, same dims).  The result tile puts
//     key l%16 and rows 4*(l/16)+i in lane l; scores are scaled after the
//     exact bf16 x bf16 products.
//   softmax over the wave's 32 keys: registers + DPP reductions inside
//     16-lane rows; p goes to LDS as [key][row].
//   PV on VALU in fp32: V in 16-byte loads, lane = 8 dims x 8 keys, the
//     four key quarters added by permlane swap butterflies (the same
//     operations for every row, whatever RMAX).
// The NW waves' (o, m, l) are merged in LDS, 8 rows at a time, and one
// unnormalised partial per row and workgroup goes to the split workspace
// (NS = ceil(L / 32 NW)).  The last workgroup of a (kv head, row tile) to
// finish -- an arrival counter per pair, bumped once the workgroup's partial
// stores have completed, wrapping back to zero on the last arrival -- merges
// the NS partials of its rows into out; no workgroup waits for another.
//
// FUSED: q holds the raw q projection rows, and the prologue does the work
// of qk_norm_rope_kv_kernel first: each wave norms and rotates whole head
// rows (qk_norm_rope_lane) -- the tile's q rows into LDS, and the new keys
// offset + t that fall in this workgroup's keys into LDS and (row tile
// 0 only) into the caches.  K / V rows of new keys come from LDS instead of
// the (possibly not yet written) cache rows.

constexpr int kDecWaveKeys = 32;  // keys per wave
constexpr int kDecMaxRows = 64;  // query rows per kv head on this path
constexpr int kMergeRows = 8;    // rows merged per LDS pass
constexpr int kFuseMaxM = 16;    // new tokens of the fused prologue
constexpr int kQS = kD + 8;      // LDS row stride of the prologue's q / k rows
// Arrival counters at the head of the workspace, one block of 512 bytes per
// (kv head, row tile): agent-scope atomics on one memory line complete one
// after another, so counters packed into one line made the arrivals of
// every kv head queue on each other.  The block's first word is the
// agent-scope counter, the word 256 bytes on the XCD-local one.
constexpr int kCounterStride = 128;                       // uints
constexpr int kMaxCounters = 64;                          // kv heads x row tiles
constexpr int kCounters = kMaxCounters * kCounterStride;  // floats
constexpr int kLocalCounter = 64;                         // uints into the block
template <int RMAX, bool FUSED, int NW>
__global__ void __launch_bounds__(64 * NW) attn_decode_kernel(const AttnParams p, const FuseParams f) {
  __shared__ __align__(16) float ps[NW][kDecWaveKeys][RMAX];
  __shared__ __align__(16) float os[NW][kMergeRows][kD];
  __shared__ float ms[NW][RMAX], ls[NW][RMAX];
  __shared__ __align__(16) uint16_t qs[FUSED ? RMAX : 1][kQS];
  __shared__ __align__(16) uint16_t kn[FUSED ? kFuseMaxM : 1][kQS];
  __shared__ __align__(16) uint16_t vn[FUSED ? kFuseMaxM : 1][kD];
  __shared__ int last;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int li = lane & 15, g = lane >> 4;
  const int tn = p.M;
  const int rep = p.Hq / p.Hkv;
  const int R = tn * rep;  // row r = j * tn + i: head kvh*rep + j, token i
  // splits in reverse launch order: the last, partly filled split goes out
  // first, so that where a CU holds two workgroups the second is a full one
  // and the short one does not queue its loads behind a full one's
  // (p.ns == gridDim.y: the split is known from the first kernel-argument
  // lines, without the round trip to the grid size behind the arguments)
  const int kvh = blockIdx.x, split = p.ns - 1 - blockIdx.y;
  const int r0 = blockIdx.z * RMAX;   // first row of this workgroup's tile
  const int RT = min(RMAX, R - r0);   // rows in the tile
  constexpr int KPS = kDecWaveKeys * NW;  // keys per split
  // ---- fused prologue, part 1: the raw rows of this wave's items -- the
  // tile's q rows, then the k / v rows of the M new tokens -- and the norm
  // weights.  None depends on the cache position, so these loads go out
  // together with the load of the position (one memory round trip for
  // both); every load is unconditional, from a valid row, so that the waits
  // for them come after the K / V stream is issued and count only these ----
  // items: it < RT: q row r0 + it; else new token it - RT
  constexpr int kItems = FUSED ? (RMAX + kFuseMaxM + NW - 1) / NW : 0;
  constexpr int kI = kItems > 0 ? kItems : 1;
  uint16_t ra[kI], rb[kI], rv0[kI], rv1[kI], wa[kI], wb[kI];
  float freq = 0.0f;
  if constexpr (FUSED) {
    // every kernel-argument field of the loads below, in one round of
    // scalar loads: left to itself the compiler requests the norm weights'
    // argument line after the first round has returned, one more memory
    // round trip ahead of every load of the launch
    asm volatile("" ::"s"(p.q), "s"(p.k), "s"(p.offset_dev), "s"(f.k_new), "s"(f.v_new), "s"(f.q_norm),
                 "s"(f.k_norm));
    freq = f.tab.inv_freq[lane];
#pragma unroll
    for (int u = 0; u < kItems; u++) {
      const int it = wave + u * NW;
      const bool is_q = it < RT;
      const int rg = r0 + min(it, RT - 1), j = rg / tn, i = rg - j * tn;
      const int64_t krow = static_cast<int64_t>(min(max(it - RT, 0), p.M - 1)) * p.Hkv + kvh;
      const uint16_t* src = is_q ? p.q + (static_cast<int64_t>(i) * p.Hq + kvh * rep + j) * kD : f.k_new + krow * kD;
      const uint16_t* nw = is_q ? f.q_norm : f.k_norm;
      ra[u] = src[lane];
      rb[u] = src[lane + 64];
      rv0[u] = f.v_new[krow * kD + lane];
      rv1[u] = f.v_new[krow * kD + lane + 64];
      wa[u] = nw[lane];
      wb[u] = nw[lane + 64];
    }
  }
  // ---- K of this workgroup's keys, issued before the cache position is
  // known (its addresses do not depend on it), through a buffer resource
  // that ends at the cache capacity: a key past the capacity reads zeros
  // without a memory access.  Keys at or beyond the L visible positions may
  // come back with any bits (rows not written yet, or this call's new rows
  // while they are written); their scores are replaced by -inf with a
  // select, never combined arithmetically, and the new rows come from LDS ----
  const int kbase = split * KPS;
  const int c0 = kbase + wave * kDecWaveKeys;
  const int64_t hbase = static_cast<int64_t>(kvh) * p.cap * kD;
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.k) + hbase, static_cast<short>(0), p.cap * kD * 2, kBufferConfig);
  uint4 kb[2][4];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    const int kofs = (c0 + t * 16 + li) * (kD * 2) + g * 16;
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      kb[t][ks] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(krs, kofs + ks * 64, 0, 0));
  }
  // the position through the constant address space: a scalar load, waited
  // for apart from the vector loads above (earlier kernels write it, this
  // one only reads it)
  const int offset =
      p.offset_dev ? *(const __attribute__((address_space(4))) int*)(p.offset_dev) : p.offset;
  if constexpr (FUSED) __builtin_amdgcn_sched_barrier(0);
  const int L = offset + p.M;
  // The grid holds a split per KPS keys of the largest context the launch
  // may see (a captured decode step: the cache capacity); only the first
  // ns_live hold keys of this call's context.  The others leave before the
  // K / V loads, and the arrival counter and the merge count only the live
  // ones, so the cost follows the context, not the capacity.  (A split
  // without visible keys contributes nothing to the merge either way:
  // results are the same bits as with every split taking part.)
  const int ns_live = min(p.ns, (L + KPS - 1) / KPS);
  if (split >= ns_live) {
    // the K loads above land before the wave ends
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }
  // this workgroup's keys: [kbase, kbase + KPS), of which those < kend exist
  const int kend = min(L, kbase + KPS);
  // new tokens whose keys fall in this workgroup's range
  const int t_lo = max(0, kbase - offset);
  const int t_hi = min(p.M, kbase + KPS - offset);
  // ---- issue loads: q fragments, K fragments, V rows ----
  uint4 qa[4];
  if constexpr (!FUSED) {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(kvh) * R + r0 + min(li, RT - 1)) * kD + g * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) qa[ks] = *reinterpret_cast<const uint4*>(qrow + ks * 32);
  }
  // V rows of this kv head through a buffer resource that ends at the L
  // visible positions: a lane whose key lies beyond them gets zeros without
  // a memory access (a raw buffer load past num_records), so a partly
  // filled split moves only its keys' V bytes, and an unweighted row is zero
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.v) + hbase, static_cast<short>(0), L * kD * 2, kBufferConfig);
  // V: lane holds dims 8 vc .. 8 vc + 7 of keys vq + 4 j, j < 8 (one 16-byte
  // load per key; an instruction reads 4 whole key rows).  With the fused
  // prologue the V loads go out after its barrier: a wave whose loads
  // outrun the CU's load queue stalls at issue, and with K and V both ahead
  // of the barrier every wave's prologue waited for the slowest issuer
  const int vc = lane & 15, vq = lane >> 4;
  uint4 vw[8];
  auto issue_v = [&]() {
#pragma unroll
    for (int j = 0; j < 8; j++)
      vw[j] = __builtin_bit_cast(
          uint4, __builtin_amdgcn_raw_buffer_load_b128(vrs, (c0 + vq + 4 * j) * (kD * 2) + 16 * vc, 0, 0));
  };
  if constexpr (!FUSED) issue_v();
  if constexpr (FUSED) {
    // ---- fused prologue, part 2: norm + rope into LDS (and the caches).
    // The rotation's cos / sin depend on the token only: a wave evaluates
    // them once per token it meets (once in all for a decode step) ----
    int ct = -1;
    float rc = 1.0f, rs = 0.0f;
#pragma unroll
    for (int u = 0; u < kItems; u++) {
      const int it = wave + u * NW;
      const bool is_q = it < RT;
      const int t = is_q ? (r0 + it) % tn : it - RT;
      if (is_q || (t >= t_lo && t < t_hi)) {
        if (t != ct) {
          rope_cs(freq, static_cast<float>(offset + t), rc, rs);
          ct = t;
        }
        uint16_t o1, o2;
        qk_norm_rope_lane_cs(bf2f(ra[u]), bf2f(rb[u]), bf2f(wa[u]), bf2f(wb[u]), rc, rs, f.eps, o1, o2);
        if (is_q) {
          qs[it][lane] = o1;
          qs[it][lane + 64] = o2;
        } else {
          kn[t][lane] = o1;
          kn[t][lane + 64] = o2;
          vn[t][lane] = rv0[u];
          vn[t][lane + 64] = rv1[u];
          if (blockIdx.z == 0) {
            // the cache rows offset + t (qwen3.rs:431-489); written once per launch
            const int64_t slot = hbase + static_cast<int64_t>(offset + t) * kD;
            uint16_t* kc = const_cast<uint16_t*>(p.k) + slot;
            uint16_t* vc = const_cast<uint16_t*>(p.v) + slot;
            kc[lane] = o1;
            kc[lane + 64] = o2;
            vc[lane] = rv0[u];
            vc[lane + 64] = rv1[u];
          }
        }
      }
    }
    __syncthreads();
    if (li < RT) {
#pragma unroll
      for (int ks = 0; ks < 4; ks++) qa[ks] = *reinterpret_cast<const uint4*>(&qs[li][ks * 32 + g * 8]);
    }
    // new keys of this split: K fragments and V rows from LDS
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int tt = c0 + t * 16 + li - offset;
      if (tt >= t_lo && tt < t_hi) {
#pragma unroll
        for (int ks = 0; ks < 4; ks++) kb[t][ks] = *reinterpret_cast<const uint4*>(&kn[tt][ks * 32 + g * 8]);
      }
    }
    issue_v();
  }
  if (li >= RT) qa[0] = qa[1] = qa[2] = qa[3] = make_uint4(0, 0, 0, 0);
  // ---- S = q K^T on MFMA ----
  f32x4_t sc[2];
#pragma unroll
  for (int t = 0; t < 2; t++) {
    sc[t] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < 4; ks++)
      sc[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, qa[ks]),
                                                      __builtin_bit_cast(bf16x8_t, kb[t][ks]), sc[t], 0, 0, 0);
  }
  // ---- softmax of the wave's 32 keys; lane holds tile rows 4g + i ----
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int r = 4 * g + i;
    if (r >= RMAX) break;
    const int rg = r0 + r;
    const int ti = rg - (rg / tn) * tn;
    const int lim = p.causal ? min(kend, offset + ti + 1) : kend;  // keys < lim are visible
    float s[2];
#pragma unroll
    for (int t = 0; t < 2; t++) s[t] = (c0 + t * 16 + li < lim) ? sc[t][i] * p.scale : -INFINITY;
    const float mx = row16_max(fmaxf(s[0], s[1]));
    float e[2];
#pragma unroll
    for (int t = 0; t < 2; t++) e[t] = (mx == -INFINITY) ? 0.0f : expf(s[t] - mx);
    const float l = row16_sum(e[0] + e[1]);
    if (r < RT) {
#pragma unroll
      for (int t = 0; t < 2; t++) ps[wave][t * 16 + li][r] = e[t];
      if (li == 0) {
        ms[wave][r] = mx;
        ls[wave][r] = l;
      }
    }
  }
  __syncthreads();
  // ---- PV ----
  // lane sums its 8 keys for every (row, dim 8 vc + d), then the four key
  // quarters (lane bits 4, 5) are added by two swap-and-add butterflies
  // (v_permlane32_swap: X' = [X.lo, Y.lo], Y' = [X.hi, Y.hi];
  // v_permlane16_swap: X' = [X.r0, Y.r0, X.r2, Y.r2], Y' = [X.r1, Y.r1, X.r3,
  // Y.r3] in 16-lane rows), which leave lane group vq with rows 4 i + vq.
  // Every row of every tile size takes the same sequence of operations, so a
  // (token, head) row's output does not depend on how many rows share the
  // launch: a verify row equals the single-token decode of the same position.
  float acc[RMAX][8];
#pragma unroll
  for (int r = 0; r < RMAX; r++)
#pragma unroll
    for (int d = 0; d < 8; d++) acc[r][d] = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) {
    // rows past the visible keys came back as zeros (never weighted either);
    // the rows of this call's new tokens come from LDS (the cache rows may
    // not be written yet)
    uint4 vj = vw[j];
    if constexpr (FUSED) {
      const int tt = c0 + vq + 4 * j - offset;
      if (tt >= t_lo && tt < t_hi) vj = *reinterpret_cast<const uint4*>(&vn[tt][8 * vc]);
    }
    const uint32_t w4[4] = {vj.x, vj.y, vj.z, vj.w};
    float v[8];
#pragma unroll
    for (int e = 0; e < 4; e++) {
      v[2 * e] = bf2f(w4[e] & 0xffffu);
      v[2 * e + 1] = bf2f(w4[e] >> 16);
    }
#pragma unroll
    for (int r4 = 0; r4 < RMAX; r4 += 4) {
      const float4 pv = *reinterpret_cast<const float4*>(&ps[wave][vq + 4 * j][r4]);
      const float pr[4] = {pv.x, pv.y, pv.z, pv.w};
#pragma unroll
      for (int q = 0; q < 4; q++)
#pragma unroll
        for (int d = 0; d < 8; d++) acc[r4 + q][d] += pr[q] * v[d];
    }
  }
#pragma unroll
  for (int i = 0; i < RMAX / 4; i++)
#pragma unroll
    for (int d = 0; d < 8; d++) {
      const auto a = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[4 * i][d]),
                                                      __float_as_uint(acc[4 * i + 2][d]), false, false);
      const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(acc[4 * i + 1][d]),
                                                      __float_as_uint(acc[4 * i + 3][d]), false, false);
      const float r1 = __uint_as_float(a[0]) + __uint_as_float(a[1]);
      const float r2 = __uint_as_float(b[0]) + __uint_as_float(b[1]);
      const auto c = __builtin_amdgcn_permlane16_swap(__float_as_uint(r1), __float_as_uint(r2), false, false);
      acc[i][d] = __uint_as_float(c[0]) + __uint_as_float(c[1]);  // row 4 i + vq, dim 8 vc + d
    }
  // ---- merge the waves kMergeRows rows at a time; thread = (row, 4 dims) ----
#pragma unroll
  for (int h0 = 0; h0 < RMAX; h0 += kMergeRows) {
    if (h0 >= RT) break;
    if (h0 > 0) __syncthreads();  // the previous pass has read os
    // rows h0 .. h0 + kMergeRows - 1 are the lane groups' rows of i = h0 / 4 ..
#pragma unroll
    for (int i2 = 0; i2 < kMergeRows / 4; i2++) {
      const int i = h0 / 4 + i2;
      if (i < RMAX / 4) {
        float* dst = &os[wave][4 * i2 + vq][8 * vc];
        *reinterpret_cast<float4*>(dst) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[i][4], acc[i][5], acc[i][6], acc[i][7]);
      }
    }
    __syncthreads();
    const int nr = min(kMergeRows, RT - h0);
    for (int e = threadIdx.x; e < nr * (kD / 4); e += 64 * NW) {
      const int rr = e / (kD / 4), d4 = e - rr * (kD / 4);
      const int r = h0 + rr;
      float m = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; w++) m = fmaxf(m, ms[w][r]);
      float l = 0.0f;
      float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (m != -INFINITY) {
#pragma unroll
        for (int w = 0; w < NW; w++) {
          if (ms[w][r] == -INFINITY) continue;
          const float a = expf(ms[w][r] - m);
          const float4 ow = *reinterpret_cast<const float4*>(&os[w][rr][d4 * 4]);
          l += a * ls[w][r];
          o.x += a * ow.x;
          o.y += a * ow.y;
          o.z += a * ow.z;
          o.w += a * ow.w;
        }
      }
      // (h * M + token) * ns + split
      const int64_t base = (static_cast<int64_t>(kvh) * R + r0 + r) * p.ns + split;
      float* po = p.part_o + base * kD + d4 * 4;
      if (p.local) {
        store_part2<true>(po, o.x, o.y);
        store_part2<true>(po + 2, o.z, o.w);
        if (d4 == 0) store_part2<true>(p.part_ml + base * 2, m, l);
      } else {
        store_part2<false>(po, o.x, o.y);
        store_part2<false>(po + 2, o.z, o.w);
        if (d4 == 0) store_part2<false>(p.part_ml + base * 2, m, l);
      }
    }
  }
  // ---- the last of the ns_live workgroups of this (kv head, row tile) merges ----
  __builtin_amdgcn_s_waitcnt(0);  // this thread's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    // Arrival: a relaxed agent-scope increment that wraps to 0 on the
    // ns_live-th arrival (ready for the next call).  Every thread's partial
    // stores (agent-coherent) completed before the barrier above; the last
    // arrival's threads read the partials with agent-coherent loads after
    // the next barrier.
    // (XCD-local: the same with the increment executed in the L2 that holds
    // the partials; their stores completed there.)
    unsigned* const c = p.cnt + (kvh * gridDim.z + blockIdx.z) * kCounterStride;
    const unsigned wrap = static_cast<unsigned>(ns_live - 1);
    if (p.local)
      last = __builtin_amdgcn_atomic_inc32(c + kLocalCounter, wrap, __ATOMIC_RELAXED, "workgroup") == wrap;
    else
      last = __builtin_amdgcn_atomic_inc32(c, wrap, __ATOMIC_RELAXED, "agent") == wrap;
  }
  __syncthreads();
  if (!last) return;
  if (p.local)
    merge_rows<NW, kL2Coherent>(p, kvh * R + r0, RT, wave, lane, ns_live);
  else
    merge_rows<NW, kAgentCoherent>(p, kvh * R + r0, RT, wave, lane, ns_live);
}

// Prefill / long verify: flash attention on MFMA.  A workgroup of 4 waves
// owns one query head and 64 consecutive query tokens (16 per wave) and
// walks the visible keys in blocks of 64 with an online softmax:
//   S^T = K Q^T (v_mfma_f32_16x16x32_bf16; A = K rows from LDS, B = the
//     wave's q rows, kept in registers) puts query l%16 and keys 4(l/16)+i
//     of each 16-key tile in lane l.  The softmax runs per lane column
//     (max / sum across the four lane quarters by shuffles), and the
//     probabilities are already an A operand for P V: over a 32-key chunk
//     lane l holds keys {4(l/16)+i} and {16+4(l/16)+i}, i < 4, which serve
//     as its 8-wide k slice in that order;
//   O += P V with B = V^T from LDS, staged transposed (4 keys x 8 dims per
//     thread, transposed in registers) so that the same 8 keys are two
//     8-byte reads.  p enters the product in fp16 against a fp16 copy of
//     V^T (one MFMA, p to 2^-11: the end-to-end logits sit at the
//     summation-order floor of the fp32 oracle with it, as with two
//     terms); a key block holding a V value beyond fp16's range (seen
//     while staging it) takes two terms instead -- bf16(p) against V in
//     bf16 plus the residual p - bf16(p) in fp16 -- and the row sums add p
//     unrounded; O and the softmax statistics are fp32.  The
//     softmax runs in base 2 (v_exp_f32 on scores pre-multiplied by log2 e),
//     and O is rescaled only in blocks where some row's running max moved.
// The K and V^T tiles are double-buffered: the loads of key block j+1 are
// issued before the products of block j.  Causal masking (query t sees keys
// <= offset + t) stops at the block holding the diagonal and masks inside.
//
// Workgroup shape <NW, HG>: NW waves of 16 queries each, over HG q heads of
// one kv head (a GQA group shares the K / V tiles) and 16 NW / HG tokens.
// The K / V loads of a key block are what bound this kernel (each CU pulls
// its tiles from L2 at a few tens of GB/s), so 8 waves over a whole group
// (4 heads x 32 tokens for Qwen3's 32 / 8 heads) halve the tile traffic per
// product against 4 waves over one head; with 8 waves, waves 0-3 stage V
// and waves 4-7 stage K.
constexpr int kFaQ = 64, kFaK = 64;  // queries per 4-wave workgroup, keys per block
constexpr int kFaKS = kD + 16;       // K tile row stride (elements)
constexpr int kFaVS = kFaK + 8;      // V^T tile row stride (elements)
// K, V^T (bf16) and V^T (fp16), double-buffered
constexpr size_t kFaLds = 2ull * (kFaK * kFaKS + 2 * kD * kFaVS) * sizeof(uint16_t);
// one bit per key block: a V value of the block lies beyond fp16's range;
// blocks past the bits (beyond 262144 keys) always take the two terms
constexpr int kFaSatWords = 128;

template <int NW, int HG>
__global__ void __launch_bounds__(64 * NW) attn_prefill_kernel(const AttnParams p) {
  static_assert((NW == 4 && HG == 1) || (NW == 8 && 8 % HG == 0), "workgroup shape");
  constexpr int TQ = 16 * NW / HG;  // tokens per workgroup
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned vsat[kFaSatWords];
  uint16_t* kt_s = reinterpret_cast<uint16_t*>(smem);  // [2][kFaK][kFaKS]
  uint16_t* vt_s = kt_s + 2 * kFaK * kFaKS;             // [2][kD][kFaVS]
  uint16_t* vh_s = vt_s + 2 * kD * kFaVS;               // [2][kD][kFaVS] fp16
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // staging: each of the 256 threads of a 4-wave workgroup stages a quarter
  // of K's rows and a 4-key x 8-dim piece of V; each of the 512 threads of
  // an 8-wave workgroup half as much (2 x 16 bytes of K, 4 keys x 4 dims of
  // V), so that every wave does the same transposition work
  const int tid = threadIdx.x & 255;
  const int n = lane & 15, g = lane >> 4;
  const int rep_h = p.Hq / p.Hkv;
  // Grid: x the head groups, y the query tiles, longest rows first (as in
  // attn_flash32_kernel: all heads' longest tiles go out first, and a head
  // group's workgroups share an XCD when there are 8 head groups).
  const int kvh = static_cast<int>(blockIdx.x) / (rep_h / HG);
  const int h = kvh * rep_h + (static_cast<int>(blockIdx.x) % (rep_h / HG)) * HG + wave % HG;
  const int t0 = (static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y)) * TQ;
  const int offset = p.offset_dev ? *p.offset_dev : p.offset;
  const int L = offset + p.M;
  const int kend = p.causal ? min(L, offset + min(t0 + TQ, p.M)) : L;
  const int nkb = (kend + kFaK - 1) / kFaK;
  const int tw = t0 + 16 * (wave / HG);  // the wave's first query
  const int t = tw + n;                  // this lane's query (softmax column)
  const int64_t hbase = static_cast<int64_t>(kvh) * p.cap * kD;

  // q fragments of the lane's query: dims 32 ks + 8 g .. + 7
  uint4 qf[4];
  {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(h) * p.M + min(t, p.M - 1)) * kD + 8 * g;
#pragma unroll
    for (int ks = 0; ks < 4; ks++) qf[ks] = *reinterpret_cast<const uint4*>(qrow + 32 * ks);
  }
  // staging of one key block: K rows (4 x 16 bytes) and V (4 keys x 8 dims);
  // plain members passed by value (no arrays or references), so the sets
  // stay in registers.  Two sets: block j + 2 is requested while block j's
  // products run and block j + 1 moves from registers into LDS.
  struct Stage {
    uint4 kr0, kr1, kr2, kr3, vr0, vr1, vr2, vr3;
  };
  const int vdc = tid & 15, vkq = tid >> 4;  // V task (4 waves): dims 8 vdc.., keys 4 vkq..
  const int vd4 = threadIdx.x & 31, vk4 = threadIdx.x >> 5;  // V task (8 waves): dims 4 vd4.., keys 4 vk4..
  auto kaddr = [&](int k0, int i) {
    const int e = (NW == 8 ? static_cast<int>(threadIdx.x) : tid) + 64 * NW * i, key = e >> 4, ch = e & 15;
    return reinterpret_cast<const uint4*>(p.k + hbase + static_cast<int64_t>(min(k0 + key, L - 1)) * kD + ch * 8);
  };
  auto vaddr = [&](int k0, int j) {
    return reinterpret_cast<const uint4*>(p.v + hbase + static_cast<int64_t>(min(k0 + 4 * vkq + j, L - 1)) * kD +
                                          vdc * 8);
  };
  auto vaddr4 = [&](int k0, int j) {
    return reinterpret_cast<const uint2*>(p.v + hbase + static_cast<int64_t>(min(k0 + 4 * vk4 + j, L - 1)) * kD +
                                          vd4 * 4);
  };
  // (with 8 waves a register set is 16 VGPRs: kr0, kr1 hold K, kr2 and kr3
  // the V rows of keys 4 vk4 .. + 3, dims 4 vd4 .. + 3)
  auto load_block = [&](int k0) {
    Stage r;
    if constexpr (NW == 8) {
      r.kr0 = *kaddr(k0, 0);
      r.kr1 = *kaddr(k0, 1);
      const uint2 v0 = *vaddr4(k0, 0), v1 = *vaddr4(k0, 1), v2 = *vaddr4(k0, 2), v3 = *vaddr4(k0, 3);
      r.kr2 = make_uint4(v0.x, v0.y, v1.x, v1.y);
      r.kr3 = make_uint4(v2.x, v2.y, v3.x, v3.y);
    } else {
      r.kr0 = *kaddr(k0, 0);
      r.kr1 = *kaddr(k0, 1);
      r.kr2 = *kaddr(k0, 2);
      r.kr3 = *kaddr(k0, 3);
      r.vr0 = *vaddr(k0, 0);
      r.vr1 = *vaddr(k0, 1);
      r.vr2 = *vaddr(k0, 2);
      r.vr3 = *vaddr(k0, 3);
    }
    return r;
  };
  auto store_block = [&](const Stage r, int buf, int blk) {
    uint16_t* kb = kt_s + buf * kFaK * kFaKS;
    auto kput = [&](int i, const uint4& v) {
      const int e = (NW == 8 ? static_cast<int>(threadIdx.x) : tid) + 64 * NW * i, key = e >> 4, ch = e & 15;
      *reinterpret_cast<uint4*>(kb + key * kFaKS + ch * 8) = v;
    };
    // V^T tiles: 4-key chunk c of dim row d sits at chunk c ^ ((d >> 3) & 7)
    // (a thread's rows share d >> 3, so the lanes of a store spread over 8
    // chunk columns instead of one bank pair).  The fp16 copy comes from
    // v_cvt_pkrtz, exact for every bf16 value in fp16's normal range and
    // saturating beyond it; a bf16 magnitude of 0x4780 (2^16) or more --
    // past fp16's largest, 65504, or inf / NaN -- marks the block for the
    // two-term product (|v| + 0x3880 carries into bit 15 of its half)
    auto h2 = [](uint32_t lo16, uint32_t hi16) {
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(lo16 << 16),
                                                                     __uint_as_float(hi16 << 16)));
    };
    auto mark = [&](uint32_t sat) {
      if (sat != 0 && blk < 32 * kFaSatWords) atomicOr(&vsat[blk >> 5], 1u << (blk & 31));
    };
    if constexpr (NW == 8) {
      kput(0, r.kr0);
      kput(1, r.kr1);
      // keys 0..3 of the piece: words (dims 4 vd4, +1) and (+2, +3)
      const uint32_t w[4][2] = {{r.kr2.x, r.kr2.y}, {r.kr2.z, r.kr2.w}, {r.kr3.x, r.kr3.y}, {r.kr3.z, r.kr3.w}};
      // saturation: the largest magnitude of each half over the 8 words
      u16x2_t mx = u16x2_t{0, 0};
#pragma unroll
      for (int k = 0; k < 4; k++)
#pragma unroll
        for (int e = 0; e < 2; e++)
          mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2_t, w[k][e] & 0x7fff7fffu));
      mark((__builtin_bit_cast(uint32_t, mx) + 0x38803880u) & 0x80008000u);
      const int cs = 4 * (vk4 ^ ((vd4 >> 1) & 7));
      uint16_t* vb = vt_s + buf * kD * kFaVS + cs;
      uint16_t* vh = vh_s + buf * kD * kFaVS + cs;
#pragma unroll
      for (int e = 0; e < 2; e++) {
        // dim rows 4 vd4 + 2 e (low halves) and + 1 (high halves): keys 0..3
        const uint32_t a = w[0][e], b = w[1][e], c = w[2][e], d = w[3][e];
        const int r0 = (4 * vd4 + 2 * e) * kFaVS, r1 = r0 + kFaVS;
        *reinterpret_cast<uint2*>(vb + r0) =
            make_uint2(__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(d, c, 0x05040100u));
        *reinterpret_cast<uint2*>(vb + r1) =
            make_uint2(__builtin_amdgcn_perm(b, a, 0x07060302u), __builtin_amdgcn_perm(d, c, 0x07060302u));
        *reinterpret_cast<uint2*>(vh + r0) = make_uint2(h2(a & 0xffffu, b & 0xffffu), h2(c & 0xffffu, d & 0xffffu));
        *reinterpret_cast<uint2*>(vh + r1) = make_uint2(h2(a >> 16, b >> 16), h2(c >> 16, d >> 16));
      }
    } else {
      kput(0, r.kr0);
      kput(1, r.kr1);
      kput(2, r.kr2);
      kput(3, r.kr3);
      const uint4 va0 = r.vr0, va1 = r.vr1, va2 = r.vr2, va3 = r.vr3;
      // V^T: dim 8 vdc + d gets keys 4 vkq .. + 3 (8 bytes)
      uint16_t* vb = vt_s + buf * kD * kFaVS + 4 * (vkq ^ (vdc & 7));
      uint16_t* vh = vh_s + buf * kD * kFaVS + 4 * (vkq ^ (vdc & 7));
      uint32_t sat = 0;
      auto chk = [&](uint32_t w) { sat |= ((w & 0x7fff7fffu) + 0x38803880u) & 0x80008000u; };
      chk(va0.x), chk(va0.y), chk(va0.z), chk(va0.w), chk(va1.x), chk(va1.y), chk(va1.z), chk(va1.w);
      chk(va2.x), chk(va2.y), chk(va2.z), chk(va2.w), chk(va3.x), chk(va3.y), chk(va3.z), chk(va3.w);
      mark(sat);
      auto vput = [&](int c, uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
        const uint2 lo = make_uint2((a0 & 0xffffu) | (a1 << 16), (a2 & 0xffffu) | (a3 << 16));
        const uint2 hi = make_uint2((a0 >> 16) | (a1 & 0xffff0000u), (a2 >> 16) | (a3 & 0xffff0000u));
        *reinterpret_cast<uint2*>(vb + (vdc * 8 + 2 * c) * kFaVS) = lo;
        *reinterpret_cast<uint2*>(vb + (vdc * 8 + 2 * c + 1) * kFaVS) = hi;
        *reinterpret_cast<uint2*>(vh + (vdc * 8 + 2 * c) * kFaVS) =
            make_uint2(h2(a0 & 0xffffu, a1 & 0xffffu), h2(a2 & 0xffffu, a3 & 0xffffu));
        *reinterpret_cast<uint2*>(vh + (vdc * 8 + 2 * c + 1) * kFaVS) =
            make_uint2(h2(a0 >> 16, a1 >> 16), h2(a2 >> 16, a3 >> 16));
      };
      vput(0, va0.x, va1.x, va2.x, va3.x);
      vput(1, va0.y, va1.y, va2.y, va3.y);
      vput(2, va0.z, va1.z, va2.z, va3.z);
      vput(3, va0.w, va1.w, va2.w, va3.w);
    }
  };

  f32x4_t o[8];
#pragma unroll
  for (int j = 0; j < 8; j++) o[j] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  float m_run = -INFINITY, l_run = 0.0f;
  const int lim = p.causal ? min(L, offset + t + 1) : L;  // keys < lim are visible to query t
  // keys below lim_w are visible to every query of the wave: a block
  // entirely below it needs no mask
  const int lim_w = p.causal ? min(L, offset + tw + 1) : L;
  const float scale2 = p.scale * 1.44269504088896340736f;  // scale * log2(e)

  Stage sg0 = load_block(0);
  Stage sg1 = load_block(min(1, nkb - 1) * kFaK);
  for (int i = threadIdx.x; i < kFaSatWords; i += 64 * NW) vsat[i] = 0u;
  __syncthreads();
  store_block(sg0, 0, 0);
  __syncthreads();
  // block jb: products from LDS buffer jb & 1; register set jb & 1 receives
  // block jb + 2 (at the end, the last block again: every iteration issues
  // the same loads, so each wait is for one specific block)
  auto iter = [&](const int jb, auto par_c) {
    constexpr int P = decltype(par_c)::value;
    const int buf = jb & 1, k0 = jb * kFaK;
    const bool more = jb + 1 < nkb;
    if constexpr (P == 0) sg0 = load_block(min(jb + 2, nkb - 1) * kFaK);
    else sg1 = load_block(min(jb + 2, nkb - 1) * kFaK);
    const uint16_t* kb = kt_s + buf * kFaK * kFaKS;
    const uint16_t* vb = vt_s + buf * kD * kFaVS;
    const uint16_t* vhb = vh_s + buf * kD * kFaVS;
    // ---- S^T = K Q^T: 4 key tiles of 16 ----
    f32x4_t sc[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
      sc[kt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < 4; ks++) {
        const uint4 a = *reinterpret_cast<const uint4*>(kb + (kt * 16 + n) * kFaKS + 32 * ks + 8 * g);
        sc[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                         __builtin_bit_cast(bf16x8_t, qf[ks]), sc[kt], 0, 0, 0);
      }
    }
    // ---- online softmax of the lane's query over the block's 64 keys, in
    // base 2: p = 2^(s c - m) with c = scale * log2(e) on v_exp_f32, the
    // scaling fused into the exponent's FMA; the running max m is of the
    // scaled scores, fl(max(s) c) = max(fl(s c)) as c > 0.  A masked key's
    // score is -inf (a select), so its p is 0 ----
    if (k0 + kFaK > lim_w) {  // uniform: the block reaches past some query's last key
#pragma unroll
      for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
          const int key = k0 + kt * 16 + 4 * g + i;
          sc[kt][i] = key < lim ? sc[kt][i] : -INFINITY;
        }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
      for (int i = 0; i < 4; i++) mx = fmaxf(mx, sc[kt][i]);
    mx = max_xor32(max_xor16(mx)) * scale2;
    const float m_new = fmaxf(m_run, mx);
    // 2^(-inf) = 0 covers the first block (m_run = -inf) and masked keys; a
    // row with nothing visible yet keeps m = -inf and is skipped
    const float m_use = m_new == -INFINITY ? 0.0f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
    // p in fp32, carried to the matrix cores in fp16 against V in fp16
    // (p to 2^-11 of itself).  A block with a V value beyond fp16's range
    // takes two terms: hi = bf16(p) against V in bf16, and the residual
    // p - hi (exact in fp32, at most 2^-9 p) rounded to fp16 against V in
    // fp16 (p to ~2^-20; a V element beyond fp16's range enters the
    // residual saturated at 65504, so its products keep hi's 2^-9).  The
    // row sum adds the unrounded p.  (One bf16
    // term, 2^-8, left the 4096-token one-layer prefill 10x further from the
    // oracle than its summation-order floor; fp16 and the two terms sit at
    // it.)
    const bool two = jb >= 32 * kFaSatWords || ((vsat[jb >> 5] >> (jb & 31)) & 1u) != 0u;
    float sum = 0.0f;
    float pv_[16];  // p of the lane's 16 keys: c, u, pair element
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const int kt = 2 * c + (u >> 1), i0 = 2 * (u & 1);
        const float r0 = __builtin_amdgcn_exp2f(fmaf(sc[kt][i0], scale2, -m_use));
        const float r1 = __builtin_amdgcn_exp2f(fmaf(sc[kt][i0 + 1], scale2, -m_use));
        sum += r0 + r1;
        pv_[8 * c + 2 * u] = r0;
        pv_[8 * c + 2 * u + 1] = r1;
      }
    bf16x8_t pa[2];
    f16x8_t pr[2];
    if (two) {  // uniform; bf16(p) and the fp16 residual only where needed
#pragma unroll
      for (int c = 0; c < 2; c++) {
        uint32_t ph[4], pl[4];
#pragma unroll
        for (int u = 0; u < 4; u++) {
          const float r0 = pv_[8 * c + 2 * u], r1 = pv_[8 * c + 2 * u + 1];
          const uint16_t b0 = f2bf(r0), b1 = f2bf(r1);
          ph[u] = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
          pl[u] = __builtin_bit_cast(
              uint32_t, f16x2_t{static_cast<_Float16>(r0 - bf2f(b0)), static_cast<_Float16>(r1 - bf2f(b1))});
        }
        pa[c] = __builtin_bit_cast(bf16x8_t, make_uint4(ph[0], ph[1], ph[2], ph[3]));
        pr[c] = __builtin_bit_cast(f16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
      }
    } else {
#pragma unroll
      for (int c = 0; c < 2; c++) {
        uint32_t pl[4];
#pragma unroll
        for (int u = 0; u < 4; u++)
          pl[u] = __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(pv_[8 * c + 2 * u]),
                                                       static_cast<_Float16>(pv_[8 * c + 2 * u + 1])});
        pa[c] = bf16x8_t{};
        pr[c] = __builtin_bit_cast(f16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
      }
    }
    sum = add_xor32(add_xor16(sum));
    l_run = l_run * alpha + sum;
    m_run = m_new;
    // ---- rescale O (rows = queries 4 g + i) when a running max moved, then
    // O += P V ----
    if (__any(alpha != 1.0f)) {
      float ar[4];
#pragma unroll
      for (int i = 0; i < 4; i++) ar[i] = __shfl(alpha, 4 * g + i, 64);
#pragma unroll
      for (int j = 0; j < 8; j++)
#pragma unroll
        for (int i = 0; i < 4; i++) o[j][i] *= ar[i];
    }
    // the fp16 product always; a block with V beyond fp16's range adds its
    // bf16 term in a second pass (one branch per block: a branch per MFMA
    // cost what the single product saves)
#pragma unroll
    for (int c = 0; c < 2; c++)
#pragma unroll
      for (int j = 0; j < 8; j++) {
        // (the scheduler may hoist the V reads of 4 dim rows at most: all
        // 16 rows' reads up front spilled registers)
        if (j % 4 == 0) __builtin_amdgcn_sched_barrier(0);
        // dim row j 16 + n, keys 32 c + 4 g.. and 32 c + 16 + 4 g.. (4-key
        // chunks 8 c + g and 8 c + 4 + g, swizzled as stored)
        const int sw = (2 * j + (n >> 3)) & 7;
        const uint16_t* hrow = vhb + (j * 16 + n) * kFaVS;
        const uint2 h0 = *reinterpret_cast<const uint2*>(hrow + 4 * ((8 * c + g) ^ sw));
        const uint2 h1 = *reinterpret_cast<const uint2*>(hrow + 4 * ((8 * c + 4 + g) ^ sw));
        const f16x8_t bh = __builtin_bit_cast(f16x8_t, make_uint4(h0.x, h0.y, h1.x, h1.y));
        o[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(pr[c], bh, o[j], 0, 0, 0);
      }
    if (two) {
#pragma unroll
      for (int c = 0; c < 2; c++)
#pragma unroll
        for (int j = 0; j < 8; j++) {
          if (j % 4 == 0) __builtin_amdgcn_sched_barrier(0);
          const int sw = (2 * j + (n >> 3)) & 7;
          const uint16_t* vrow = vb + (j * 16 + n) * kFaVS;
          const uint2 v0 = *reinterpret_cast<const uint2*>(vrow + 4 * ((8 * c + g) ^ sw));
          const uint2 v1 = *reinterpret_cast<const uint2*>(vrow + 4 * ((8 * c + 4 + g) ^ sw));
          const bf16x8_t bv = __builtin_bit_cast(bf16x8_t, make_uint4(v0.x, v0.y, v1.x, v1.y));
          o[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa[c], bv, o[j], 0, 0, 0);
        }
    }
    if (more) store_block(P == 0 ? sg1 : sg0, buf ^ 1, jb + 1);
    __syncthreads();
  };
  for (int jb = 0; jb < nkb; jb += 2) {
    iter(jb, std::integral_constant<int, 0>{});
    if (jb + 1 < nkb) iter(jb + 1, std::integral_constant<int, 1>{});
  }
  // ---- normalise and write: lane holds dim 16 j + n of queries 4 g + i ----
  float lr[4];
#pragma unroll
  for (int i = 0; i < 4; i++) lr[i] = __shfl(l_run, 4 * g + i, 64);
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int tq = tw + 4 * g + i;
    if (tq >= p.M) continue;
    const float inv = lr[i] > 0.0f ? 1.0f / lr[i] : 0.0f;
    uint16_t* orow = p.out + static_cast<int64_t>(tq) * p.Hq * kD + h * kD + n;
#pragma unroll
    for (int j = 0; j < 8; j++) orow[16 * j] = f2bf(o[j][i] * inv);
  }
}

// Prefill / long verify with 32 queries per wave (v_mfma_f32_32x32x16):
// the same staging, LDS tiles, online softmax and V-range guard as
// attn_prefill_kernel<8, HG>, arranged so that each query's softmax state
// stays in one lane.  A workgroup of 8 waves owns HG q heads of one kv head
// and 256 / HG consecutive tokens, 32 per wave.  Per 64-key block:
//   S^T = K Q^T on v_mfma_f32_32x32x16_bf16 (A = 32 keys of the K tile, B =
//     the wave's q rows, 16 dims a step): lane l holds query l % 32 and
//     keys 32 kt + 8 (r / 4) + 4 (l / 32) + r % 4 of the two key tiles kt;
//     row max and sum run over the lane's 32 scores and the other half of
//     the wave (one lane swap);
//   O^T += V^T P^T on v_mfma_f32_32x32x16_f16 (A = 32 dims of V^T from LDS,
//     two 4-key chunks per lane; B = the probabilities as they lie in the
//     score registers: keys 16 s + 4 (l / 32) + 0..3 and + 8 of step s are
//     eight consecutive score registers), so O^T puts query l % 32 in lane
//     l as well, and its rescale by exp(m_old - m_new) needs no shuffle.
// Half the LDS operand reads per product of the 16-query layout, and the
// cross-lane reductions of a block halve.
typedef __attribute__((ext_vector_type(16))) float f32x16_t;
// Its LDS rows (strides chosen with a bank-conflict probe of each access:
// 16-byte operand reads of 32 consecutive rows are conflict-free at 272
// bytes for K and at 192 bytes with the (d >> 3) & 7 pair swizzle for V^T)
constexpr int kF32KS = kD + 8;   // K tile row stride (elements)
constexpr int kF32VS = kFaK + 32;  // V^T tile row stride (elements)
constexpr size_t kF32Lds = 2ull * (kFaK * kF32KS + 2 * kD * kF32VS) * sizeof(uint16_t);

template <int HG>
__global__ void __launch_bounds__(512) attn_flash32_kernel(const AttnParams p) {
  constexpr int NW = 8;
  constexpr int TQ = 32 * NW / HG;  // tokens per workgroup
  extern __shared__ __align__(16) unsigned char smem[];
  __shared__ unsigned vsat[kFaSatWords];
  uint16_t* kt_s = reinterpret_cast<uint16_t*>(smem);  // [2][kFaK][kF32KS]
  uint16_t* vt_s = kt_s + 2 * kFaK * kF32KS;            // [2][kD][kF32VS]
  uint16_t* vh_s = vt_s + 2 * kD * kF32VS;              // [2][kD][kF32VS] fp16
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = lane & 31, hf = lane >> 5;  // query column, lane half
  const int rep_h = p.Hq / p.Hkv;
  // Grid: x the head groups, y the query tiles, longest rows first.  The
  // hardware hands out workgroups in linear order (x fastest), so every
  // head's longest tiles go out before any shorter one, and with 8 head
  // groups workgroup b's XCD (b % 8) is that of its head group: one kv
  // head's K / V stays in one L2.
  const int kvh = static_cast<int>(blockIdx.x) / (rep_h / HG);
  const int h = kvh * rep_h + (static_cast<int>(blockIdx.x) % (rep_h / HG)) * HG + wave % HG;
  const int t0 = (static_cast<int>(gridDim.y) - 1 - static_cast<int>(blockIdx.y)) * TQ;
  const int offset = p.offset_dev ? *p.offset_dev : p.offset;
  const int L = offset + p.M;
  const int kend = p.causal ? min(L, offset + min(t0 + TQ, p.M)) : L;
  const int nkb = (kend + kFaK - 1) / kFaK;
  const int tw = t0 + 32 * (wave / HG);  // the wave's first query
  const int t = tw + j;                  // this lane's query
  const int64_t hbase = static_cast<int64_t>(kvh) * p.cap * kD;

  // q of the lane's query: dims 16 ks + 8 hf .. + 7 (B of S^T = K Q^T)
  uint4 qf[8];
  {
    const uint16_t* qrow = p.q + (static_cast<int64_t>(h) * p.M + min(t, p.M - 1)) * kD + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < 8; ks++) qf[ks] = *reinterpret_cast<const uint4*>(qrow + 16 * ks);
  }
  // staging of one key block by the 512 threads: K rows (2 x 16 bytes) and V
  // (4 keys x 4 dims, transposed in registers), as attn_prefill_kernel<8, .>
  struct Stage {
    uint4 kr0, kr1, kr2, kr3;
  };
  // V piece of a thread: dims 4 vd4 .. + 3, keys 4 vk4 .. + 3.  Lanes 0-15
  // and 32-47 of a wave read one 256-byte key row, lanes 16-31 and 48-63 the
  // row 8 keys on, and the V^T stores below fall in distinct LDS banks.
  const int tid9 = static_cast<int>(threadIdx.x);
  const int vd4 = (tid9 & 15) | (((tid9 >> 5) & 1) << 4);
  const int vk4 = (((tid9 >> 4) & 1) << 1) | ((tid9 >> 6) & 1) | ((tid9 >> 7) << 2);
  auto kaddr = [&](int k0, int i) {
    const int e = static_cast<int>(threadIdx.x) + 512 * i, key = e >> 4, ch = e & 15;
    return reinterpret_cast<const uint4*>(p.k + hbase + static_cast<int64_t>(min(k0 + key, L - 1)) * kD + ch * 8);
  };
  auto vaddr4 = [&](int k0, int jj) {
    return reinterpret_cast<const uint2*>(p.v + hbase + static_cast<int64_t>(min(k0 + 4 * vk4 + jj, L - 1)) * kD +
                                          vd4 * 4);
  };
  auto load_block = [&](int k0) {
    Stage r;
    r.kr0 = *kaddr(k0, 0);
    r.kr1 = *kaddr(k0, 1);
    const uint2 v0 = *vaddr4(k0, 0), v1 = *vaddr4(k0, 1), v2 = *vaddr4(k0, 2), v3 = *vaddr4(k0, 3);
    r.kr2 = make_uint4(v0.x, v0.y, v1.x, v1.y);
    r.kr3 = make_uint4(v2.x, v2.y, v3.x, v3.y);
    return r;
  };
  auto store_block = [&](const Stage r, int buf, int blk) {
    uint16_t* kb = kt_s + buf * kFaK * kF32KS;
    auto kput = [&](int i, const uint4& v) {
      const int e = static_cast<int>(threadIdx.x) + 512 * i, key = e >> 4, ch = e & 15;
      *reinterpret_cast<uint4*>(kb + key * kF32KS + ch * 8) = v;
    };
    // V^T: a dim row holds its 64 keys as 8 pairs of 4-key chunks, pair P =
    // 2 g + (c & 1) holding chunks c and c + 2 of 16-key group g (keys
    // 16 g + 4 c.. ), so the 8 keys a lane feeds one P V product are 16
    // contiguous bytes; pair P of dim row d sits at P ^ ((d >> 3) & 7).
    // fp16 copy by v_cvt_pkrtz (exact in fp16's normal range); a bf16
    // magnitude of 2^16 or more marks the block for the two-term product
    auto h2 = [](uint32_t lo16, uint32_t hi16) {
      return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__uint_as_float(lo16 << 16),
                                                                     __uint_as_float(hi16 << 16)));
    };
    kput(0, r.kr0);
    kput(1, r.kr1);
    const uint32_t w[4][2] = {{r.kr2.x, r.kr2.y}, {r.kr2.z, r.kr2.w}, {r.kr3.x, r.kr3.y}, {r.kr3.z, r.kr3.w}};
    u16x2_t mx = u16x2_t{0, 0};
#pragma unroll
    for (int k = 0; k < 4; k++)
#pragma unroll
      for (int e = 0; e < 2; e++) mx = __builtin_elementwise_max(mx, __builtin_bit_cast(u16x2_t, w[k][e] & 0x7fff7fffu));
    const uint32_t sat = (__builtin_bit_cast(uint32_t, mx) + 0x38803880u) & 0x80008000u;
    if (sat != 0 && blk < 32 * kFaSatWords) atomicOr(&vsat[blk >> 5], 1u << (blk & 31));
    const int cs = 8 * ((2 * (vk4 >> 2) + (vk4 & 1)) ^ ((vd4 >> 1) & 7)) + 4 * ((vk4 >> 1) & 1);
    uint16_t* vb = vt_s + buf * kD * kF32VS + cs;
    uint16_t* vh = vh_s + buf * kD * kF32VS + cs;
#pragma unroll
    for (int e = 0; e < 2; e++) {
      const uint32_t a = w[0][e], b = w[1][e], c = w[2][e], d = w[3][e];
      const int r0 = (4 * vd4 + 2 * e) * kF32VS, r1 = r0 + kF32VS;
      *reinterpret_cast<uint2*>(vb + r0) =
          make_uint2(__builtin_amdgcn_perm(b, a, 0x05040100u), __builtin_amdgcn_perm(d, c, 0x05040100u));
      *reinterpret_cast<uint2*>(vb + r1) =
          make_uint2(__builtin_amdgcn_perm(b, a, 0x07060302u), __builtin_amdgcn_perm(d, c, 0x07060302u));
      *reinterpret_cast<uint2*>(vh + r0) = make_uint2(h2(a & 0xffffu, b & 0xffffu), h2(c & 0xffffu, d & 0xffffu));
      *reinterpret_cast<uint2*>(vh + r1) = make_uint2(h2(a >> 16, b >> 16), h2(c >> 16, d >> 16));
    }
  };

  f32x16_t o[4];  // O^T: dims 32 dt + 8 (r / 4) + 4 hf + r % 4 of query t
#pragma unroll
  for (int dt = 0; dt < 4; dt++)
#pragma unroll
    for (int r = 0; r < 16; r++) o[dt][r] = 0.0f;
  float m_run = -INFINITY, l_run = 0.0f;
  const int lim = p.causal ? min(L, offset + t + 1) : L;       // keys < lim are visible to query t
  const int lim_w = p.causal ? min(L, offset + tw + 1) : L;    // ... to every query of the wave
  const int lim_hi = p.causal ? min(L, offset + tw + 32) : L;  // ... to some query of the wave
  const float scale2 = p.scale * 1.44269504088896340736f;      // scale * log2(e)
  // V^T reads: dim row d = 32 dt + j, pair P = 2 s + hf (keys 16 s + 4 hf
  // .. and 16 s + 8 + 4 hf ..), at pair P ^ ((d >> 3) & 7).  The swizzle's
  // bits are (j >> 3) & 1, (j >> 4) & 1 and dt & 1, so the position is a
  // lane part for each parity of s plus constants:
  //   P ^ sw = (hf ^ sw0) + 2 ((s & 1) ^ sw1) + 4 ((s >> 1) ^ (dt & 1))
  const int sw0 = (j >> 3) & 1, sw1 = (j >> 4) & 1;
  const int vle = j * kF32VS + 8 * ((hf ^ sw0) + 2 * sw1);        // s even
  const int vlo = j * kF32VS + 8 * ((hf ^ sw0) + 2 * (1 - sw1));  // s odd
  auto vaddr = [&](int dt, int s) {
    return ((s & 1) ? vlo : vle) + 32 * dt * kF32VS + 32 * ((s >> 1) ^ (dt & 1));
  };

  // two register sets: block jb + 2 is requested while block jb's products
  // run and block jb + 1 moves from registers into LDS
  Stage sg0 = load_block(0);
  Stage sg1 = load_block(min(1, nkb - 1) * kFaK);
  for (int i = threadIdx.x; i < kFaSatWords; i += 512) vsat[i] = 0u;
  __syncthreads();
  store_block(sg0, 0, 0);
  __syncthreads();
  auto iter = [&](const int jb, auto par_c) {
    constexpr int P = decltype(par_c)::value;
    const int buf = jb & 1, k0 = jb * kFaK;
    const bool more = jb + 1 < nkb;
    if constexpr (P == 0) sg0 = load_block(min(jb + 2, nkb - 1) * kFaK);
    else sg1 = load_block(min(jb + 2, nkb - 1) * kFaK);
    if (k0 < lim_hi) {  // uniform per wave: some query of the wave sees a key of this block
      const uint16_t* kb = kt_s + buf * kFaK * kF32KS;
      const uint16_t* vb = vt_s + buf * kD * kF32VS;
      const uint16_t* vhb = vh_s + buf * kD * kF32VS;
      // ---- S^T = K Q^T: 2 key tiles of 32, 8 dim steps of 16 ----
      f32x16_t sc[2];
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) sc[kt][r] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < 8; ks++)
#pragma unroll
        for (int kt = 0; kt < 2; kt++) {
          // (K reads hoisted one dim step at most: registers)
          if (kt == 0) __builtin_amdgcn_sched_barrier(0);
          const uint4 a = *reinterpret_cast<const uint4*>(kb + (kt * 32 + j) * kF32KS + 16 * ks + 8 * hf);
          sc[kt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                           __builtin_bit_cast(bf16x8_t, qf[ks]), sc[kt], 0, 0, 0);
        }
      // ---- online softmax of query t over the block, base 2 (as the
      // 16-query kernel: p = 2^(s c - m), masked keys -inf by a select) ----
      if (k0 + kFaK > lim_w) {  // uniform: the block reaches past some query's last key
#pragma unroll
        for (int kt = 0; kt < 2; kt++)
#pragma unroll
          for (int r = 0; r < 16; r++) {
            const int key = k0 + 32 * kt + 8 * (r >> 2) + 4 * hf + (r & 3);
            sc[kt][r] = key < lim ? sc[kt][r] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) mx = fmaxf(mx, sc[kt][r]);
      mx = max_xor32(mx) * scale2;
      const float m_new = fmaxf(m_run, mx);
      const float m_use = m_new == -INFINITY ? 0.0f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
      const bool two = jb >= 32 * kFaSatWords || ((vsat[jb >> 5] >> (jb & 31)) & 1u) != 0u;
      float sum = 0.0f;
#pragma unroll
      for (int kt = 0; kt < 2; kt++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
          const float e = __builtin_amdgcn_exp2f(fmaf(sc[kt][r], scale2, -m_use));
          sum += e;
          sc[kt][r] = e;
        }
      sum = add_xor32(sum);
      l_run = l_run * alpha + sum;
      m_run = m_new;
      // ---- rescale O^T where a running max moved (each lane its own query) ----
      if (__any(alpha != 1.0f)) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++)
#pragma unroll
          for (int r = 0; r < 16; r++) o[dt][r] *= alpha;
      }
      // ---- O^T += V^T P^T: key step s = registers 8 (s & 1) .. + 7 of tile
      // s / 2.  p in fp16 against V in fp16; a block holding a V value beyond
      // fp16's range takes p = hi + lo instead, hi = bf16(p) against V in bf16
      // and lo = p - hi (exact in fp32) in fp16 against V in fp16 (saturated
      // there) ----
      f16x8_t ph[4];
      bf16x8_t pa[4];
      if (two) {  // uniform; bf16(p) and the fp16 residual only where needed
#pragma unroll
        for (int s = 0; s < 4; s++) {
          uint32_t hw[4], lw[4];
#pragma unroll
          for (int u = 0; u < 4; u++) {
            const float r0 = sc[s >> 1][8 * (s & 1) + 2 * u], r1 = sc[s >> 1][8 * (s & 1) + 2 * u + 1];
            const uint16_t b0 = f2bf(r0), b1 = f2bf(r1);
            hw[u] = static_cast<uint32_t>(b0) | (static_cast<uint32_t>(b1) << 16);
            lw[u] = __builtin_bit_cast(
                uint32_t, f16x2_t{static_cast<_Float16>(r0 - bf2f(b0)), static_cast<_Float16>(r1 - bf2f(b1))});
          }
          pa[s] = __builtin_bit_cast(bf16x8_t, make_uint4(hw[0], hw[1], hw[2], hw[3]));
          ph[s] = __builtin_bit_cast(f16x8_t, make_uint4(lw[0], lw[1], lw[2], lw[3]));
        }
      } else {
#pragma unroll
        for (int s = 0; s < 4; s++) {
          uint32_t pl[4];
#pragma unroll
          for (int u = 0; u < 4; u++)
            pl[u] = __builtin_bit_cast(uint32_t, f16x2_t{static_cast<_Float16>(sc[s >> 1][8 * (s & 1) + 2 * u]),
                                                         static_cast<_Float16>(sc[s >> 1][8 * (s & 1) + 2 * u + 1])});
          ph[s] = __builtin_bit_cast(f16x8_t, make_uint4(pl[0], pl[1], pl[2], pl[3]));
          pa[s] = bf16x8_t{};
        }
      }
      // the fp16 product always; a block with V beyond fp16's range adds its
      // bf16 term in a second pass
#pragma unroll
      for (int dt = 0; dt < 4; dt++) {
        __builtin_amdgcn_sched_barrier(0);  // (V reads of one dim tile at a time)
#pragma unroll
        for (int s = 0; s < 4; s++) {
          const uint4 hv = *reinterpret_cast<const uint4*>(vhb + vaddr(dt, s));
          o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8_t, hv), ph[s], o[dt], 0, 0, 0);
        }
      }
      if (two) {
#pragma unroll
        for (int dt = 0; dt < 4; dt++) {
          __builtin_amdgcn_sched_barrier(0);
#pragma unroll
          for (int s = 0; s < 4; s++) {
            const uint4 vv = *reinterpret_cast<const uint4*>(vb + vaddr(dt, s));
            o[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, vv), pa[s], o[dt], 0, 0, 0);
          }
        }
      }
    }
    if (more) store_block(P == 0 ? sg1 : sg0, buf ^ 1, jb + 1);
    __syncthreads();
  };
  for (int jb = 0; jb < nkb; jb += 2) {
    iter(jb, std::integral_constant<int, 0>{});
    if (jb + 1 < nkb) iter(jb + 1, std::integral_constant<int, 1>{});
  }
  // ---- normalise and write: dims 32 dt + 8 r4 + 4 hf .. + 3 of query t ----
  if (t < p.M) {
    const float inv = l_run > 0.0f ? 1.0f / l_run : 0.0f;
    uint16_t* orow = p.out + static_cast<int64_t>(t) * p.Hq * kD + h * kD + 4 * hf;
#pragma unroll
    for (int dt = 0; dt < 4; dt++)
#pragma unroll
      for (int r4 = 0; r4 < 4; r4++) {
        const f32x16_t& a = o[dt];
        const uint32_t w0 = static_cast<uint32_t>(f2bf(a[4 * r4] * inv)) |
                            (static_cast<uint32_t>(f2bf(a[4 * r4 + 1] * inv)) << 16);
        const uint32_t w1 = static_cast<uint32_t>(f2bf(a[4 * r4 + 2] * inv)) |
                            (static_cast<uint32_t>(f2bf(a[4 * r4 + 3] * inv)) << 16);
        *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * r4) = make_uint2(w0, w1);
      }
  }
}

}  // namespace

// Workspace floats of one call: the arrival counters, then the split
// partials.
size_t attention_workspace_floats(int Hq, int M, int ns) {
  return kCounters + static_cast<size_t>(Hq) * M * ns * (kD + 2);
}

namespace {

// ---- where the workgroups of a launch run: the XCD-local merge's premise ----
// xcd_probe_kernel records the XCD (hardware register XCC_ID) of every
// workgroup of a grid shaped like the decode kernel's (x = 8 kv heads);
// the merge may stay in one L2 when every workgroup with the same x runs on
// one XCD.  Checked once per device, at the first uncaptured call.
constexpr int kProbeX = 8, kProbeY = 24, kProbeZ = 3;  // 576 workgroups
constexpr int kProbeWgs = kProbeX * kProbeY * kProbeZ;
constexpr int kMaxDevices = 64;

__device__ __align__(256) unsigned xcd_probe_out[kProbeWgs];

__global__ void __launch_bounds__(64) xcd_probe_kernel(unsigned* out) {
  // s_getreg_b32 of XCC_ID (hardware register 20), bits 0-3
  if (threadIdx.x == 0)
    out[blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z)] =
        __builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 15u;
}

std::mutex g_xcd_mu;
signed char g_xcd_local[kMaxDevices];  // 0 unchecked, 1 holds, -1 does not

bool xcd_local_ok(hipStream_t stream) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
    (void)hipGetLastError();
    return false;
  }
  std::lock_guard<std::mutex> lock(g_xcd_mu);
  if (g_xcd_local[dev]) return g_xcd_local[dev] > 0;
  // not under capture: the check waits for its result (a later call checks)
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  if (cs != hipStreamCaptureStatusNone) return false;
  void* ptr = nullptr;
  unsigned host[kProbeWgs];
  bool ok = hipGetSymbolAddress(&ptr, HIP_SYMBOL(xcd_probe_out)) == hipSuccess;
  if (ok) {
    hipLaunchKernelGGL(xcd_probe_kernel, dim3(kProbeX, kProbeY, kProbeZ), dim3(64), 0, stream,
                       static_cast<unsigned*>(ptr));
    ok = hipGetLastError() == hipSuccess &&
         hipMemcpyAsync(host, ptr, sizeof host, hipMemcpyDeviceToHost, stream) == hipSuccess &&
         hipStreamSynchronize(stream) == hipSuccess;
  }
  if (!ok) (void)hipGetLastError();
  for (int i = 0; ok && i < kProbeWgs; i++) ok = host[i] == host[i % kProbeX];
  g_xcd_local[dev] = ok ? 1 : -1;
  return ok;
}

// The split-key decode path, if the call fits it: R = M * rep <= 64 rows per
// kv head, a workspace with room for one split per 256 keys, and (fused) at
// most kFuseMaxM new tokens.  Returns kNoFit when it does not apply.
int launch_decode(const AttnParams& base, const FuseParams* fuse, float* ws, size_t ws_floats, int L_max,
                  hipStream_t stream) {
  const int Hq = base.Hq, Hkv = base.Hkv, M = base.M;
  const int rep = Hq / Hkv, R = M * rep;
  if (!ws || R > kDecMaxRows || (fuse && M > kFuseMaxM)) return kNoFit;
  if (!aligned(ws, 16)) return set_error(BMX_E_ALIGN, "attention: workspace must be 16-byte aligned");
  if (ws_floats < kCounters) return kNoFit;
  const int max_ns = static_cast<int>((ws_floats - kCounters) / (static_cast<size_t>(Hq) * M * (kD + 2)));
  // row tiles of 4 (decode: up to 4 q heads per kv head) or 8 rows; a
  // 16-row tile (half the workgroups for R > 8, each re-reading K and V
  // fewer times, but twice the PV registers and work per wave) measured
  // slower: 32B-shape verify step 9.53 against 9.26 ms with 8-row tiles;
  // 4-row tiles throughout, 9.41 ms
  const int rmax = R <= 4 ? 4 : 8;
  const int tiles = (R + rmax - 1) / rmax;
  // Keys per split: 32 per wave, 8 waves (256 keys).  Splits of 128 keys
  // (4 waves: a 4K context over all CUs, 33 splits per kv head against 17)
  // measured slower in the decode step at context 4096: 12.93 against 12.15
  // us per layer -- the data phase shortens by ~1 us, but twice as many
  // arrivals serialize on each kv head's counter (~0.1 us apiece).  The
  // split size is fixed, so every row of a cache (decode or verify) is
  // partitioned alike.
  const int nw = 8;
  const int kps = kDecWaveKeys * nw;
  const int chunks = (L_max + kps - 1) / kps;
  if (chunks > max_ns) return kNoFit;
  if (Hkv * tiles > kMaxCounters) return kNoFit;
  AttnParams p = base;
  p.cnt = reinterpret_cast<unsigned*>(ws);
  p.part_o = ws + kCounters;
  p.part_ml = p.part_o + static_cast<size_t>(Hq) * M * chunks * kD;
  p.tq = M;
  p.ns = chunks;
  p.kps = kps;
  p.causal = M > 1 ? 1 : 0;
  // x = kv head: with a multiple of 8 kv heads, every workgroup of a kv
  // head shares the XCD of its x
  p.local = Hkv % 8 == 0 && xcd_local_ok(stream);
  const FuseParams f = fuse ? *fuse : FuseParams{};
  const dim3 grid(Hkv, chunks, tiles), block(64 * nw);
#define BMX_DECODE_LAUNCH(RM, NW)                                                        \
  do {                                                                                   \
    if (fuse)                                                                            \
      hipLaunchKernelGGL((attn_decode_kernel<RM, true, NW>), grid, block, 0, stream, p, f);  \
    else                                                                                 \
      hipLaunchKernelGGL((attn_decode_kernel<RM, false, NW>), grid, block, 0, stream, p, f); \
  } while (0)
  if (rmax == 4 && nw == 4)
    BMX_DECODE_LAUNCH(4, 4);
  else if (rmax == 4)
    BMX_DECODE_LAUNCH(4, 8);
  else if (nw == 4)
    BMX_DECODE_LAUNCH(8, 4);
  else
    BMX_DECODE_LAUNCH(8, 8);
#undef BMX_DECODE_LAUNCH
  return check_launch(fuse ? "attention_decode_fused" : "attention_decode");
}

int check_attention_shape(int Hq, int Hkv, int M, int D, int cap, int offset, const int* offset_dev) {
  if (D != kD) return set_error(BMX_E_UNSUPPORTED, "attention: head_dim must be 128 (got %d)", D);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || M <= 0) return set_error(BMX_E_SHAPE, "attention: bad head counts");
  if (!offset_dev && (offset < 0 || offset + M > cap))
    return set_error(BMX_E_KV_CAPACITY, "attention: %d positions exceed capacity %d", offset + M, cap);
  return BMX_OK;
}

}  // namespace

void attention_prepare(hipStream_t stream) { (void)xcd_local_ok(stream); }

int launch_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, float* ws,
                     size_t ws_floats, int Hq, int Hkv, int M, int D, int cap, int offset, const int* offset_dev,
                     int L_max, float scale, hipStream_t stream) {
  if (int rc = check_attention_shape(Hq, Hkv, M, D, cap, offset, offset_dev)) return rc;
  AttnParams p{q, k, v, out, nullptr, nullptr, nullptr, offset_dev, offset, Hq, Hkv, M, cap, kFaQ, 1,
               M > 1 ? 1 : 0, scale};
  const int rc = launch_decode(p, nullptr, ws, ws_floats, L_max, stream);
  if (rc != kNoFit) return rc;
  // flash attention (no split workspace): a GQA group per workgroup when
  // the heads per kv head are a power of two, else one head per workgroup
  const int rep = Hq / Hkv;
  auto launch = [&](auto kern, int nw, int hg) {
    if (int e = allow_lds_ptr(reinterpret_cast<const void*>(kern), kFaLds)) return e;
    const int tq = 16 * nw / hg, tiles = (M + tq - 1) / tq;
    if (tiles > 65535) return set_error(BMX_E_SHAPE, "attention: M=%d too large for one prefill launch", M);
    hipLaunchKernelGGL(kern, dim3(Hkv * (rep / hg), tiles), dim3(64 * nw), kFaLds, stream, p);
    return check_launch("attention_prefill");
  };
  auto launch32 = [&](auto kern, int hg) {
    if (int e = allow_lds_ptr(reinterpret_cast<const void*>(kern), kF32Lds)) return e;
    const int tq = 256 / hg, tiles = (M + tq - 1) / tq;
    if (tiles > 65535) return set_error(BMX_E_SHAPE, "attention: M=%d too large for one prefill launch", M);
    hipLaunchKernelGGL(kern, dim3(Hkv * (rep / hg), tiles), dim3(512), kF32Lds, stream, p);
    return check_launch("attention_prefill");
  };
  if (rep % 8 == 0) return launch32(attn_flash32_kernel<8>, 8);
  if (rep == 4) return launch32(attn_flash32_kernel<4>, 4);
  if (rep == 2) return launch32(attn_flash32_kernel<2>, 2);
  if (rep == 1) return launch32(attn_flash32_kernel<1>, 1);
  return launch(attn_prefill_kernel<4, 1>, 4, 1);
}

int launch_qkv_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                         const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, float* ws,
                         size_t ws_floats, int Hq, int Hkv, int M, int D, int cap, int offset,
                         const int* offset_dev, int L_max, float eps, const RopeTable& tab, float scale,
                         hipStream_t stream) {
  if (int rc = check_attention_shape(Hq, Hkv, M, D, cap, offset, offset_dev)) return rc;
  AttnParams p{q, k_cache, v_cache, out, nullptr, nullptr, nullptr, offset_dev, offset, Hq, Hkv, M, cap, M, 1,
               M > 1 ? 1 : 0, scale};
  FuseParams f{k, v, q_norm, k_norm, eps, tab};
  return launch_decode(p, &f, ws, ws_floats, L_max, stream);
}

}  // namespace bmx

using namespace bmx;

extern "C" size_t bmx_attention_workspace_bytes(int n_heads, int M) {
  // enough for one split per 256 keys of a 65536-position cache
  return attention_workspace_floats(n_heads, M, 256) * sizeof(float);
}

extern "C" int bmx_attention_gqa(const bmx_bf16* q, const bmx_bf16* k_cache, const bmx_bf16* v_cache, bmx_bf16* out,
                                 int n_heads, int n_kv_heads, int M, int head_dim, int capacity, int offset,
                                 float scale, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !out) return set_error(BMX_E_ARG, "attention: null pointer");
  return launch_attention(q, k_cache, v_cache, out, static_cast<float*>(workspace), workspace_bytes / sizeof(float),
                          n_heads, n_kv_heads, M, head_dim, capacity, offset, nullptr, offset + M, scale,
                          as_stream(stream));
}

extern "C" int bmx_qk_norm_rope_kv_attention(const bmx_bf16* q, const bmx_bf16* k, const bmx_bf16* v,
                                             const bmx_bf16* q_norm, const bmx_bf16* k_norm, bmx_bf16* k_cache,
                                             bmx_bf16* v_cache, bmx_bf16* out, int M, int n_heads, int n_kv_heads,
                                             int head_dim, int capacity, int offset, float eps, float theta,
                                             float scale, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !q_norm || !k_norm || !k_cache || !v_cache || !out || !workspace)
    return set_error(BMX_E_ARG, "qk_norm_rope_kv_attention: null pointer");
  const int rc = launch_qkv_attention(q, k, v, q_norm, k_norm, k_cache, v_cache, out, static_cast<float*>(workspace),
                                      workspace_bytes / sizeof(float), n_heads, n_kv_heads, M, head_dim, capacity,
                                      offset, nullptr, offset + M, eps, make_rope_table(head_dim, theta), scale,
                                      as_stream(stream));
  if (rc == kNoFit)
    return set_error(BMX_E_UNSUPPORTED,
                     "qk_norm_rope_kv_attention: needs M <= %d, M * (n_heads / n_kv_heads) <= %d and a workspace of "
                     "bmx_attention_workspace_bytes(n_heads, M) bytes",
                     kFuseMaxM, kDecMaxRows);
  return rc;
}
