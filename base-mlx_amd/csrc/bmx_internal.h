// Host-side internals shared by the bmx translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>
#include <vector>

#include "bmx.h"

namespace bmx {

// Records a message for bmx_last_error() and returns `code`.
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Converts the last HIP launch status into a bmx return code (0 or a
// positive hipError_t) and records its message.
int check_launch(const char* what);
int check_hip(hipError_t e, const char* what);

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// ---- qmv (M <= 8) -------------------------------------------------------
enum QmvEpilogue { QMV_STORE = 0, QMV_RESIDUAL = 1, QMV_SWIGLU = 2 };

struct QmvSegment {
  const uint32_t* w;  // [rows, K/8]
  const uint16_t* s;  // [rows, K/64]
  const uint16_t* b;  // [rows, K/64]
  uint16_t* y;        // [M, rows] (row stride = rows)
  int rows;
  int row0;  // first global output row of this segment
  int blk0;  // first workgroup of this segment (set by launch_qmv)
};

struct QmvParams {
  const uint16_t* x;  // [M, K], row stride ldx
  int64_t ldx;
  QmvSegment seg[3];
  int nseg;
  int m;  // rows of x (1..8)
  int N;  // total output rows over all segments (SWIGLU: rows of one matrix)
  int K;
  const uint16_t* res;     // QMV_RESIDUAL: [M, N] added to the product (may alias y)
  const uint16_t* norm_w;  // optional fused RMSNorm of x: weight [K]
  float eps;
  int kp;      // K columns staged in LDS per phase (set by launch_qmv)
  int sb_vec;  // s/b staged with 16-byte loads (set by launch_qmv)
  // QMV_STORE with one segment: optional per-workgroup argmax partials of
  // the bf16 outputs, (value bits, row) at [m * qmv_blocks(...) + workgroup]
  uint2* amax;
  // optional workspace for the K-split matrix-core GEMV (fp32 partials);
  // without one the library's buffer of the stream is used
  float* part;
  size_t part_floats;
};

// Raises a kernel's dynamic-LDS limit to `bytes` (launches above 64 KB need
// it); returns a BMX code.  Limits already raised are remembered per kernel.
int allow_lds_ptr(const void* kernel, size_t bytes);
// Workgroups of `threads` threads and `lds` bytes of dynamic LDS that the
// current device holds at once (per-CU occupancy x CUs).
int resident_blocks(const void* kernel, int threads, size_t lds);
template <class F>
int allow_lds(F* kernel, size_t bytes) {
  if (bytes <= 64 * 1024) return BMX_OK;
  return allow_lds_ptr(reinterpret_cast<const void*>(kernel), bytes);
}

// Validates shapes/alignment and launches the qmv kernel family.
int launch_qmv(QmvParams p, QmvEpilogue epi, hipStream_t stream);
// Matrices (N output rows, K columns) the matrix-core GEMV takes for every
// row count 1..8; all other shapes take the dot2 GEMV kernels.  Argmax
// partials come from the dot2 kernels only.
bool qmv_mfma_family(int N, int K);
// The matrix-core GEMV; kNoFit when the shape does not fit it (a function of
// the shape, never of the row count).
int try_launch_qmvx(QmvParams p, QmvEpilogue epi, hipStream_t stream);
// Partial floats the K-split matrix-core GEMV needs for M rows of x and an
// N x K weight (0 if it never splits that shape).
size_t qmvx_workspace_floats(int M, int N, int K);
// Workgroups launch_qmv uses for these parameters (the count of argmax
// partials per x row).
int qmv_blocks(const QmvParams& p, QmvEpilogue epi);

// ---- other kernels (one launch each, errors recorded) --------------------
// Dequantizing MFMA GEMM (M > 8).  Split-K partials go to ws when it holds
// qmm_workspace_floats of the shape, else to a buffer of the (device,
// stream) pair that the library keeps.
int launch_qmm(const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b, uint16_t* y, int M,
               int N, int K, float* ws, size_t ws_floats, hipStream_t stream);
// The same x times up to 3 weights (q, k, v of a layer) with separate
// outputs y[i] of n[i] columns: one launch when every n[i] is a multiple of
// 128 and K does not split, else one launch_qmm per weight.  Each output is
// bit-identical to its own launch_qmm without a K split.
int launch_qmm_segments(const uint16_t* x, int nseg, const uint32_t* const* w, const uint16_t* const* s,
                        const uint16_t* const* b, uint16_t* const* y, const int* n, int M, int K, float* ws,
                        size_t ws_floats, hipStream_t stream);
// The GEMM with a fused epilogue: store; residual, y = res + bf16(x W^T)
// (res may alias y); SwiGLU of the gate W and up W2 weights,
// y = bf16(silu(bf16(x W^T)) * bf16(x W2^T)) with MLX's roundings.  SwiGLU
// returns kNoFit (nothing launched) when the shape would split K.
enum QmmEpilogue { QMM_STORE = 0, QMM_RESIDUAL = 1, QMM_SWIGLU = 2, QMM_QKV_ROPE = 3 };
int launch_qmm_epi(QmmEpilogue epi, const uint16_t* x, const uint32_t* w, const uint16_t* s, const uint16_t* b,
                   const uint32_t* w2, const uint16_t* s2, const uint16_t* b2, const uint16_t* res, uint16_t* y, int M,
                   int N, int K, float* ws, size_t ws_floats, hipStream_t stream);
// The same products over group-major copies of the weights (launch_qmm_repack):
// W as [K/64][N][8] words and s|b as [K/64][N] words s | b << 16, so the
// rows of one group in a tile are contiguous.  Bit-identical to the MLX-layout
// launches; kNoFit (nothing launched) where the one-launch segments form or
// the SwiGLU form does not fit, for the caller's MLX-layout fallback.
int launch_qmm_epi_gm(QmmEpilogue epi, const uint16_t* x, const uint32_t* w, const uint32_t* sb, const uint32_t* w2,
                      const uint32_t* sb2, const uint16_t* res, uint16_t* y, int M, int N, int K, float* ws,
                      size_t ws_floats, hipStream_t stream);
int launch_qmm_segments_gm(const uint16_t* x, int nseg, const uint32_t* const* w, const uint32_t* const* sb,
                           uint16_t* const* y, const int* n, int M, int K, float* ws, size_t ws_floats,
                           hipStream_t stream);
// Writes the group-major copy (wt: N * K / 8 words, sbt: N * K / 64 words)
// of an MLX-layout weight w, s, b of N rows by K.
int launch_qmm_repack(const uint32_t* w, const uint16_t* s, const uint16_t* b, int N, int K, uint32_t* wt,
                      uint32_t* sbt, hipStream_t stream);
// Split-K partial floats the GEMM needs for any M up to max_M (0 if none).
size_t qmm_workspace_floats(int max_M, int N, int K);
// A device buffer of at least `floats` floats owned by the library for the
// (device, stream) pair, grown on demand (growing synchronizes the stream);
// work on one stream runs in order, so its launches may share it.
int stream_scratch(size_t floats, hipStream_t stream, float** out);
// Split-K partials of `need` floats: the caller's workspace ws when given
// (an error when it holds fewer than `need`), else -- unless a NoAllocScope
// is active on this thread, which makes it an error -- stream_scratch.
int split_scratch(size_t need, float* ws, size_t ws_floats, hipStream_t stream, float** out);
// While an object of this type lives, split_scratch never allocates on the
// calling thread (entry points that must not allocate).
struct NoAllocScope {
  NoAllocScope();
  ~NoAllocScope();
  NoAllocScope(const NoAllocScope&) = delete;
  NoAllocScope& operator=(const NoAllocScope&) = delete;
};
// Split-K partial floats one GEMM call of this epilogue and shape uses (0
// when K is not split).
size_t qmm_need_floats(QmmEpilogue epi, int M, int N, int K);
int launch_rms_norm(const uint16_t* x, const uint16_t* w, uint16_t* y, int64_t rows, int dim, float eps,
                    hipStream_t stream);
struct RopeTable {
  float inv_freq[128];  // theta^(-i/(D/2)), i < D/2 <= 128, evaluated in double
};
RopeTable make_rope_table(int D, float theta);
int launch_qk_norm_rope_kv(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                           const uint16_t* k_norm, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache, int M,
                           int Hq, int Hkv, int D, int cap, int offset, const int* offset_dev, float eps,
                           const RopeTable& tab, hipStream_t stream);
// (cos, sin) of the rotation of M tokens at positions offset + t (or
// *offset_dev + t), frequency i < 64 at cs[t * 64 + i]: the values the
// QK-norm / RoPE kernels compute per token (head_dim 128)
int launch_rope_cs(float2* cs, int M, int offset, const int* offset_dev, const RopeTable& tab, hipStream_t stream);
// Outputs of the q|k|v GEMM with the QK-norm / RoPE / KV-write epilogue
// (the operation of launch_qk_norm_rope_kv, head_dim 128): q rotated into
// q_out [Hq, M, 128], k rotated and v into the caches [Hkv, cap, 128] at
// rows offset + t; cs from launch_rope_cs
struct QkvRopeOut {
  const uint16_t* q_norm;
  const uint16_t* k_norm;
  uint16_t* q_out;
  uint16_t* k_cache;
  uint16_t* v_cache;
  const float2* cs;
  const int* offset_dev;
  int offset;
  int cap;
  float eps;
};
// The q|k|v GEMM (group-major weights, segments q, k, v of n[i] columns,
// whole 128-column head tiles) with that epilogue; kNoFit where the GEMM
// would split K or take 256-column tiles (nothing launched).
int launch_qmm_qkv_rope_gm(const uint16_t* x, const uint32_t* const* w, const uint32_t* const* sb, const int* n,
                           int M, int K, const QkvRopeOut& out, hipStream_t stream);
// A weight tensor of a bmx_qwen3 under its MLX checkpoint name: rows x cols
// of uint32 (packed 4-bit weights) or bf16 (scales, biases, norm weights).
struct WeightSlot {
  std::string name;
  void* dev;
  int rows, cols;
  bool u32;
};
// Allocates a Qwen3 of shape cfg (weights uninitialised) with its forward
// workspace; every weight tensor, named as in an MLX checkpoint.
int qwen3_alloc(const bmx_qwen3_config* cfg, int max_tokens, bmx_qwen3** out);
std::vector<WeightSlot> qwen3_weight_slots(bmx_qwen3* m);

// Returned by a launcher whose kernel does not fit the call (nothing launched).
constexpr int kNoFit = -100;
// Attention workspace (floats): arrival counters, then split partials; the
// counters must be zero before the first call, and every call leaves them so.
size_t attention_workspace_floats(int Hq, int M, int ns);
// Runs the decode kernel's one-time device check (waits for the stream);
// call before capturing a graph that holds decode attention.
void attention_prepare(hipStream_t stream);
// QK-norm + RoPE + KV write + decode attention in one kernel; kNoFit unless
// M <= 16, M * (Hq / Hkv) <= 64 and ws holds one split per 256 keys of L_max.
int launch_qkv_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, const uint16_t* q_norm,
                         const uint16_t* k_norm, uint16_t* k_cache, uint16_t* v_cache, uint16_t* out, float* ws,
                         size_t ws_floats, int Hq, int Hkv, int M, int D, int cap, int offset,
                         const int* offset_dev, int L_max, float eps, const RopeTable& tab, float scale,
                         hipStream_t stream);
int launch_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, float* ws,
                     size_t ws_floats, int Hq, int Hkv, int M, int D, int cap, int offset, const int* offset_dev,
                     int L_max, float scale, hipStream_t stream);
// The hand-off between decode steps queued back to back: io = [token,
// position, next token, ring count] in device memory, ring = `mask + 1`
// slots of mapped host memory.  A one-row argmax given a chain writes its
// token to io[0] (the next step's embedding id), advances io[1] (the next
// step's position) and stores the token to ring[io[3]++ & mask].
struct DecodeChain {
  int* io = nullptr;
  uint32_t* ring = nullptr;
  unsigned mask = 0;
};
int launch_argmax(const uint16_t* x, int64_t rows, int64_t n, uint32_t* out, hipStream_t stream,
                  const DecodeChain* chain = nullptr);
// Reduces `nblk` argmax partials per row (from the qmv epilogue) to out[rows].
int launch_argmax_partials(const uint2* part, int rows, int nblk, uint32_t* out, hipStream_t stream,
                           const DecodeChain* chain = nullptr);
int launch_silu_mul(const uint16_t* g, const uint16_t* u, uint16_t* y, int64_t n, hipStream_t stream);
int launch_add(const uint16_t* a, const uint16_t* b, uint16_t* y, int64_t n, hipStream_t stream);
int launch_tokens_to_ids(const uint32_t* src, int32_t* dst, int n, hipStream_t stream);
int launch_dequant_gather(const int32_t* ids, int64_t M, int64_t rows, const uint32_t* w, const uint16_t* s,
                          const uint16_t* b, uint16_t* out, int64_t K, hipStream_t stream);
int launch_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c, uint32_t* w, uint16_t* s, uint16_t* b,
                        hipStream_t stream);
int launch_fill_kv_synthetic(uint16_t* data, int64_t rows, int cap, int hd, int seq_len, uint64_t seed, float c,
                             hipStream_t stream);
uint64_t host_mix64(uint64_t z);

}  // namespace bmx
