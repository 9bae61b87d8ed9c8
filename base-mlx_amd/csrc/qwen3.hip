// Qwen3 forward, KV cache, greedy and speculative generation over the bmx
// kernels: the host side of the drop-in, mirroring the reference's model
// and engine surface.
//
//   bmx_qwen3_*          <-> Qwen3 { load, forward, forward_multi }
//                            (crates/base-mlx-core/src/model/qwen3.rs:164-563)
//   bmx_kv_*             <-> KvCache { reset, truncate, seq_len }
//                            (qwen3.rs:109-162)
//   bmx_generate_greedy  <-> LoadedModel::generate_text with greedy pick_next
//                            (crates/base-mlx-core/src/engine.rs:100-202)
//   bmx_decode_greedy    <-> its decode loop alone, after the prefill
//                            (engine.rs:103-115)
//   bmx_speculative_generate <-> speculative::generate
//                            (crates/base-mlx-core/src/speculative.rs:57-286)
//
// Device layout.  Each projection keeps the MLX format (W [N, K/8] u32,
// s/b [N, K/64] bf16).  The KV cache is one buffer [L, 2, Hkv, cap, 128]
// bf16 (the reference's per-layer [Hkv, KV_PREALLOC, 128] pairs, capacity a
// parameter); truncate rewinds seq_len and keeps the buffer, as the comment
// at qwen3.rs:146-149 intends.
//
// Per layer at M <= 8 (decode, verify): one qmv for q|k|v with the input
// RMSNorm fused, one fused QK-norm + RoPE + KV write, attention (+ split
// combine), o_proj qmv with the residual add fused, gate|up qmv with the
// post-attention RMSNorm and SwiGLU fused, down qmv with the residual add
// fused.  At M > 8 (prefill) the norms, SwiGLU and adds run as their own
// kernels around the MFMA qmm.  The M = 1 decode step is captured once per
// cache into a HIP graph that reads the token and position from device
// memory and leaves the next ones there, so a decode step is one graph
// launch and the greedy loop queues steps without waiting for each token.
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <vector>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr double kIrwin4Std = 37837.226523565;  // sqrt((65536^2 - 1) / 3)
enum { SLOT_Q, SLOT_K, SLOT_V, SLOT_O, SLOT_GATE, SLOT_UP, SLOT_DOWN, NSLOT };

struct QLin {
  uint32_t* w = nullptr;
  uint16_t* s = nullptr;
  uint16_t* b = nullptr;
  int N = 0, K = 0;
  // the group-major copy the prefill GEMMs read (layer projections;
  // launch_qmm_repack): W [K/64][N][8] words, s|b [K/64][N] words
  uint32_t* wt = nullptr;
  uint32_t* sbt = nullptr;
};

struct Layer {
  QLin p[NSLOT];
  uint16_t *in_norm = nullptr, *post_norm = nullptr, *q_norm = nullptr, *k_norm = nullptr;
};

uint64_t tensor_seed(uint64_t model_seed, int layer, int slot) {
  return host_mix64(model_seed * 0xD1B54A32D192ED03ull + static_cast<uint64_t>(static_cast<int64_t>(layer + 16)) * 64u +
                    static_cast<uint64_t>(slot));
}

__global__ void fill_ones_kernel(uint16_t* p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0x3f80;
}

}  // namespace
}  // namespace bmx

using namespace bmx;

// Decode steps in flight: the host ring the decode graph publishes tokens to
// (a power of two), how many replays the greedy loop queues ahead of the
// token it is checking, and the value of a slot not yet written.
constexpr int kRing = 64;
constexpr int kAhead = 3;
constexpr uint32_t kRingEmpty = 0xffffffffu;
// verify width of speculative decoding (leader + drafts), at most
constexpr int kMaxSpecK = 8;
// forwards of more tokens than this norm and rotate q / k in the q|k|v GEMM
// (more than 64 query rows per kv head: the attention is the flash kernel,
// which reads the rotated rows, never the fused decode kernel)
constexpr int kRopeGemmMinM = 64;

struct bmx_kv_cache {
  uint64_t id = 0;  // unique per cache: keys the captured decode graph
  int layers = 0, nkv = 0, hd = 0, cap = 0;
  int seq_len = 0;
  uint16_t* data = nullptr;  // [layers, 2, nkv, cap, hd]
  uint16_t* k(int l) { return data + static_cast<size_t>(l) * 2 * nkv * cap * hd; }
  uint16_t* v(int l) { return k(l) + static_cast<size_t>(nkv) * cap * hd; }
};

struct bmx_qwen3 {
  bmx_qwen3_config cfg{};
  int max_tokens = 0;
  QLin embed, lm_head;
  uint16_t* final_norm = nullptr;
  std::vector<Layer> layers;
  RopeTable rope{};
  float2* rope_cs = nullptr;  // (cos, sin) of a long forward's positions (launch_rope_cs)
  std::vector<void*> allocs;
  // workspace (rows = max_tokens)
  uint16_t *x = nullptr, *h = nullptr, *q = nullptr, *k = nullptr, *v = nullptr, *qr = nullptr, *att = nullptr,
           *o = nullptr, *g = nullptr, *u = nullptr, *a = nullptr, *logits1 = nullptr;
  uint16_t* vlogits = nullptr;  // [kMaxSpecK, vocab]: a speculative verify forward's logits
  float* attn_ws = nullptr;
  size_t attn_ws_floats = 0;
  float* qmm_ws = nullptr;  // split-K partials of the prefill GEMMs (per model: models on
  size_t qmm_ws_floats = 0;  // different streams never share one)
  int32_t* ids = nullptr;     // [max_tokens] token ids for the embedding gather
  uint32_t* tok_u = nullptr;  // [max(max_tokens, 64)] token staging
  uint32_t* next_tok = nullptr;  // argmax output of the decode step
  int* step_io = nullptr;        // decode graph: [token, position, next token, ring count] (device)
  uint32_t* ring = nullptr;      // mapped host [kRing]: tokens the decode graph publishes
  uint32_t* ring_dev = nullptr;  // the same memory, as the device addresses it
  uint2* amax = nullptr;         // lm_head argmax partials of the decode graph
  int amax_cap = 0;
  uint32_t* host_tok = nullptr;    // pinned [64]: token / position / argmax exchange
  uint32_t* host_stage = nullptr;  // pinned [max_tokens]: prompt upload staging
  hipEvent_t stage_done = nullptr; // host_stage may be rewritten once this fired
  hipStream_t own_stream = nullptr;  // used when the caller passes the null stream
  // the layer projections' group-major copies must be rewritten before the
  // next GEMM reads them
  bool gm_stale = true;
  // decode graph
  hipGraphExec_t graph = nullptr;
  uint64_t graph_cache = 0;  // id of the cache the graph was captured for
  hipStream_t graph_stream = nullptr;
};

namespace {

int dalloc(bmx_qwen3* m, void** p, size_t bytes) {
  if (bytes == 0) bytes = 16;
  hipError_t e = hipMalloc(p, bytes);
  if (e != hipSuccess) return set_error(BMX_E_ALLOC, "hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
  m->allocs.push_back(*p);
  return BMX_OK;
}

template <typename T>
int dalloc_t(bmx_qwen3* m, T** p, size_t count) {
  return dalloc(m, reinterpret_cast<void**>(p), count * sizeof(T));
}

int alloc_qlin(bmx_qwen3* m, QLin* q, int N, int K, bool group_major = false) {
  q->N = N;
  q->K = K;
  if (int rc = dalloc_t(m, &q->w, static_cast<size_t>(N) * (K / 8))) return rc;
  if (int rc = dalloc_t(m, &q->s, static_cast<size_t>(N) * (K / 64))) return rc;
  if (int rc = dalloc_t(m, &q->b, static_cast<size_t>(N) * (K / 64))) return rc;
  if (!group_major) return BMX_OK;
  if (int rc = dalloc_t(m, &q->wt, static_cast<size_t>(N) * (K / 8))) return rc;
  return dalloc_t(m, &q->sbt, static_cast<size_t>(N) * (K / 64));
}

// Rewrites every group-major copy from its MLX-layout weight (after the
// weights are set, or after a caller was handed pointers it may have
// written through)
int repack_prefill_weights(bmx_qwen3* m, hipStream_t st) {
  for (Layer& L : m->layers)
    for (QLin& q : L.p)
      if (q.wt)
        if (int rc = launch_qmm_repack(q.w, q.s, q.b, q.N, q.K, q.wt, q.sbt, st)) return rc;
  m->gm_stale = false;
  return BMX_OK;
}

int fill_ones(uint16_t* p, int n, hipStream_t st) {
  hipLaunchKernelGGL(fill_ones_kernel, dim3((n + 255) / 256), dim3(256), 0, st, p, n);
  return check_launch("fill_ones");
}

int qmv(const bmx_qwen3* m, const uint16_t* x, int M, const QLin& w, uint16_t* y, hipStream_t st,
        const uint16_t* norm = nullptr, uint2* amax = nullptr, int* amax_nblk = nullptr) {
  QmvParams p{};
  p.x = x;
  p.ldx = w.K;
  p.nseg = 1;
  p.seg[0] = QmvSegment{w.w, w.s, w.b, y, w.N, 0};
  p.m = M;
  p.N = w.N;
  p.K = w.K;
  p.norm_w = norm;
  p.eps = m->cfg.eps;
  // the matrix-core GEMV (large heads) writes no argmax partials: the
  // caller then reduces the logits row itself (*amax_nblk = 0)
  if (amax && qmv_mfma_family(w.N, w.K)) {
    amax = nullptr;
    if (amax_nblk) *amax_nblk = 0;
  }
  p.amax = amax;
  if (amax) {
    const int nblk = qmv_blocks(p, QMV_STORE);
    if (nblk > m->amax_cap) return set_error(BMX_E_SHAPE, "argmax partials: %d workgroups", nblk);
    if (amax_nblk) *amax_nblk = nblk;
  }
  return launch_qmv(p, QMV_STORE, st);
}

const QLin& head_of(const bmx_qwen3* m) { return m->cfg.tied ? m->embed : m->lm_head; }

// One forward over M tokens whose ids are already in m->ids, at position
// cache->seq_len (or *pos_dev when graph-captured).  logits: [rows, vocab]
// (rows = M if all_logits else 1).
// ids: token ids on device (m->ids when null).  amax (one logits row only):
// the head GEMV also writes its argmax partials there, *amax_nblk of them.
int forward_device(bmx_qwen3* m, bmx_kv_cache* c, int M, int offset, const int* pos_dev, bool all_logits,
                   uint16_t* logits, hipStream_t st, const int32_t* ids = nullptr, uint2* amax = nullptr,
                   int* amax_nblk = nullptr) {
  const bmx_qwen3_config& cf = m->cfg;
  const int H = cf.hidden, I = cf.inter, nq = cf.n_heads, nkv = cf.n_kv_heads, hd = cf.head_dim;
  const int qd = nq * hd, kvd = nkv * hd;
  const float scale = 1.0f / sqrtf(static_cast<float>(hd));  // qwen3.rs:324
  const int L_max = pos_dev ? c->cap : offset + M;
  if (M > 8 && m->gm_stale) {
    if (int rc = repack_prefill_weights(m, st)) return rc;
  }
  // long forwards norm and rotate q / k in the q|k|v GEMM's epilogue (the
  // attention then takes the flash kernel, which reads them from q_out and
  // the caches); the rotation's (cos, sin) once per forward
  const bool rope_gemm = M > kRopeGemmMinM && hd == 128;
  if (rope_gemm) {
    if (int rc = launch_rope_cs(m->rope_cs, M, offset, pos_dev, m->rope, st)) return rc;
  }
  // x = embed.lookup(tokens)  (qwen3.rs:328-333)
  if (int rc = launch_dequant_gather(ids ? ids : m->ids, M, cf.vocab, m->embed.w, m->embed.s, m->embed.b, m->x, H, st))
    return rc;
  for (int l = 0; l < cf.layers; l++) {
    const Layer& L = m->layers[l];
    bool roped = false;  // q / k normed and rotated, caches written, by the q|k|v GEMM
    // ---- qkv_block: rms_norm + q/k/v projections (kernels.rs:28-46) ----
    if (M <= 8) {
      QmvParams p{};
      p.x = m->x;
      p.ldx = H;
      p.nseg = 3;
      p.seg[0] = QmvSegment{L.p[SLOT_Q].w, L.p[SLOT_Q].s, L.p[SLOT_Q].b, m->q, qd, 0};
      p.seg[1] = QmvSegment{L.p[SLOT_K].w, L.p[SLOT_K].s, L.p[SLOT_K].b, m->k, kvd, qd};
      p.seg[2] = QmvSegment{L.p[SLOT_V].w, L.p[SLOT_V].s, L.p[SLOT_V].b, m->v, kvd, qd + kvd};
      p.m = M;
      p.N = qd + 2 * kvd;
      p.K = H;
      p.norm_w = L.in_norm;
      p.eps = cf.eps;
      if (int rc = launch_qmv(p, QMV_STORE, st)) return rc;
    } else {
      if (int rc = launch_rms_norm(m->x, L.in_norm, m->h, M, H, cf.eps, st)) return rc;
      // q, k and v in one GEMM launch where the shape allows (qwen3.rs:370-390)
      const uint32_t* wt3[3] = {L.p[SLOT_Q].wt, L.p[SLOT_K].wt, L.p[SLOT_V].wt};
      const uint32_t* sb3[3] = {L.p[SLOT_Q].sbt, L.p[SLOT_K].sbt, L.p[SLOT_V].sbt};
      uint16_t* y3[3] = {m->q, m->k, m->v};
      const int n3[3] = {qd, kvd, kvd};
      int rc = kNoFit;
      if (rope_gemm) {
        const QkvRopeOut ro{L.q_norm, L.k_norm, m->qr, c->k(l), c->v(l), m->rope_cs, pos_dev, offset, c->cap, cf.eps};
        rc = launch_qmm_qkv_rope_gm(m->h, wt3, sb3, n3, M, H, ro, st);
        if (rc == BMX_OK) roped = true;
      }
      if (rc == kNoFit) rc = launch_qmm_segments_gm(m->h, 3, wt3, sb3, y3, n3, M, H, m->qmm_ws, m->qmm_ws_floats, st);
      if (rc == kNoFit) {
        const uint32_t* w3[3] = {L.p[SLOT_Q].w, L.p[SLOT_K].w, L.p[SLOT_V].w};
        const uint16_t* s3[3] = {L.p[SLOT_Q].s, L.p[SLOT_K].s, L.p[SLOT_V].s};
        const uint16_t* b3[3] = {L.p[SLOT_Q].b, L.p[SLOT_K].b, L.p[SLOT_V].b};
        rc = launch_qmm_segments(m->h, 3, w3, s3, b3, y3, n3, M, H, m->qmm_ws, m->qmm_ws_floats, st);
      }
      if (rc) return rc;
    }
    // ---- QK-norm, RoPE at the cache offset, KV write (qwen3.rs:392-489) and
    // SDPA over [0, offset + M) with the causal-offset mask (qwen3.rs:491-518):
    // one fused kernel for decode / short verify, else two steps ----
    const int fused = roped ? kNoFit
                            : launch_qkv_attention(m->q, m->k, m->v, L.q_norm, L.k_norm, c->k(l), c->v(l), m->att,
                                                   m->attn_ws, m->attn_ws_floats, nq, nkv, M, hd, c->cap, offset,
                                                   pos_dev, L_max, cf.eps, m->rope, scale, st);
    if (fused != kNoFit) {
      if (fused) return fused;
    } else {
      if (!roped) {
        if (int rc = launch_qk_norm_rope_kv(m->q, m->k, m->v, L.q_norm, L.k_norm, m->qr, c->k(l), c->v(l), M, nq,
                                            nkv, hd, c->cap, offset, pos_dev, cf.eps, m->rope, st))
          return rc;
      }
      if (int rc = launch_attention(m->qr, c->k(l), c->v(l), m->att, m->attn_ws, m->attn_ws_floats, nq, nkv, M, hd,
                                    c->cap, offset, pos_dev, L_max, scale, st))
        return rc;
    }
    // ---- o_proj + residual (qwen3.rs:520-521) ----
    if (M <= 8) {
      QmvParams p{};
      p.x = m->att;
      p.ldx = qd;
      p.nseg = 1;
      p.seg[0] = QmvSegment{L.p[SLOT_O].w, L.p[SLOT_O].s, L.p[SLOT_O].b, m->x, H, 0};
      p.m = M;
      p.N = H;
      p.K = qd;
      p.res = m->x;
      p.part = m->qmm_ws;
      p.part_floats = m->qmm_ws_floats;
      if (int rc = launch_qmv(p, QMV_RESIDUAL, st)) return rc;
    } else {
      if (int rc = launch_qmm_epi_gm(QMM_RESIDUAL, m->att, L.p[SLOT_O].wt, L.p[SLOT_O].sbt, nullptr, nullptr, m->x,
                                     m->x, M, H, qd, m->qmm_ws, m->qmm_ws_floats, st))
        return rc;
    }
    // ---- mlp_block + residual (kernels.rs:55-78; qwen3.rs:523-541) ----
    if (M <= 8) {
      QmvParams p{};
      p.x = m->x;
      p.ldx = H;
      p.nseg = 2;
      p.seg[0] = QmvSegment{L.p[SLOT_GATE].w, L.p[SLOT_GATE].s, L.p[SLOT_GATE].b, m->a, I, 0};
      p.seg[1] = QmvSegment{L.p[SLOT_UP].w, L.p[SLOT_UP].s, L.p[SLOT_UP].b, m->a, I, 0};
      p.m = M;
      p.N = I;
      p.K = H;
      p.norm_w = L.post_norm;
      p.eps = cf.eps;
      if (int rc = launch_qmv(p, QMV_SWIGLU, st)) return rc;
      QmvParams d{};
      d.x = m->a;
      d.ldx = I;
      d.nseg = 1;
      d.seg[0] = QmvSegment{L.p[SLOT_DOWN].w, L.p[SLOT_DOWN].s, L.p[SLOT_DOWN].b, m->x, H, 0};
      d.m = M;
      d.N = H;
      d.K = I;
      d.res = m->x;
      d.part = m->qmm_ws;
      d.part_floats = m->qmm_ws_floats;
      if (int rc = launch_qmv(d, QMV_RESIDUAL, st)) return rc;
    } else {
      if (int rc = launch_rms_norm(m->x, L.post_norm, m->h, M, H, cf.eps, st)) return rc;
      // gate, up and SwiGLU in one GEMM when it does not split K, else three steps
      const QLin &gw = L.p[SLOT_GATE], &uw = L.p[SLOT_UP];
      const int fused = launch_qmm_epi_gm(QMM_SWIGLU, m->h, gw.wt, gw.sbt, uw.wt, uw.sbt, nullptr, m->a, M, I, H,
                                          m->qmm_ws, m->qmm_ws_floats, st);
      if (fused != kNoFit) {
        if (fused) return fused;
      } else {
        if (int rc = launch_qmm(m->h, gw.w, gw.s, gw.b, m->g, M, I, H, m->qmm_ws, m->qmm_ws_floats, st)) return rc;
        if (int rc = launch_qmm(m->h, uw.w, uw.s, uw.b, m->u, M, I, H, m->qmm_ws, m->qmm_ws_floats, st)) return rc;
        if (int rc = launch_silu_mul(m->g, m->u, m->a, static_cast<int64_t>(M) * I, st)) return rc;
      }
      if (int rc = launch_qmm_epi_gm(QMM_RESIDUAL, m->a, L.p[SLOT_DOWN].wt, L.p[SLOT_DOWN].sbt, nullptr, nullptr, m->x,
                                     m->x, M, H, I, m->qmm_ws, m->qmm_ws_floats, st))
        return rc;
    }
  }
  // ---- final norm, last row unless all logits, tied head (qwen3.rs:545-555) ----
  const QLin& head = head_of(m);
  const int rows = all_logits ? M : 1;
  const uint16_t* xin = all_logits ? m->x : m->x + static_cast<size_t>(M - 1) * H;
  if (rows <= 8) return qmv(m, xin, rows, head, logits, st, m->final_norm, rows == 1 ? amax : nullptr, amax_nblk);
  if (int rc = launch_rms_norm(xin, m->final_norm, m->h, rows, H, cf.eps, st)) return rc;
  return launch_qmm(m->h, head.w, head.s, head.b, logits, rows, cf.vocab, H, m->qmm_ws, m->qmm_ws_floats, st);
}

// Decode step with token and position in device memory (step_io[0], [1]):
// forward, with the lm_head GEMV writing per-workgroup argmax partials, then
// the reduction of the partials -> step_io[2].  Captured into a graph.  The
// token is read as the embedding id directly: tokens are below the
// vocabulary size (checked on the host, or produced by the argmax).  The
// argmax also hands the step over to the next one (DecodeChain): the token
// becomes step_io[0], the position step_io[1] + 1, and the token lands in
// ring slot step_io[3]++ -- so replays queued back to back decode
// consecutive tokens without the host in between.
int decode_step_device(bmx_qwen3* m, bmx_kv_cache* c, hipStream_t st) {
  int nblk = 0;
  if (int rc = forward_device(m, c, 1, 0, m->step_io + 1, false, m->logits1, st, m->step_io, m->amax, &nblk))
    return rc;
  uint32_t* next = reinterpret_cast<uint32_t*>(m->step_io + 2);
  const DecodeChain chain{m->step_io, m->ring_dev, kRing - 1};
  if (nblk == 0) return launch_argmax(m->logits1, 1, m->cfg.vocab, next, st, &chain);
  return launch_argmax_partials(m->amax, 1, nblk, next, st, &chain);
}

void drop_graph(bmx_qwen3* m) {
  if (m->graph) (void)hipGraphExecDestroy(m->graph);
  m->graph = nullptr;
  m->graph_cache = 0;
}

int ensure_graph(bmx_qwen3* m, bmx_kv_cache* c, hipStream_t st) {
  if (m->graph && m->graph_cache == c->id && m->graph_stream == st) return BMX_OK;
  drop_graph(m);
  hipGraph_t g = nullptr;
  if (int rc = check_hip(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal), "begin capture")) return rc;
  int rc = decode_step_device(m, c, st);
  hipError_t e = hipStreamEndCapture(st, &g);
  if (rc) {
    if (g) (void)hipGraphDestroy(g);
    return rc;
  }
  if (int r2 = check_hip(e, "end capture")) return r2;
  e = hipGraphInstantiate(&m->graph, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (int r2 = check_hip(e, "graph instantiate")) return r2;
  m->graph_cache = c->id;
  m->graph_stream = st;
  return BMX_OK;
}

bool is_eos(uint32_t t, const uint32_t* eos, int n_eos) {
  for (int i = 0; i < n_eos; i++)
    if (eos[i] == t) return true;
  return false;
}

// tokens (host) -> m->ids (device) through the pinned staging buffer
int upload_tokens(bmx_qwen3* m, const uint32_t* tokens, int M, hipStream_t st) {
  for (int i = 0; i < M; i++)
    if (tokens[i] >= static_cast<uint32_t>(m->cfg.vocab))
      return set_error(BMX_E_ARG, "token %u at %d outside vocab %d", tokens[i], i, m->cfg.vocab);
  if (int rc = check_hip(hipEventSynchronize(m->stage_done), "stage wait")) return rc;
  memcpy(m->host_stage, tokens, static_cast<size_t>(M) * 4);
  if (int rc = check_hip(hipMemcpyAsync(m->tok_u, m->host_stage, static_cast<size_t>(M) * 4, hipMemcpyHostToDevice, st),
                         "upload tokens"))
    return rc;
  if (int rc = check_hip(hipEventRecord(m->stage_done, st), "stage record")) return rc;
  return launch_tokens_to_ids(m->tok_u, m->ids, M, st);
}

hipStream_t pick_stream(bmx_qwen3* m, void* stream) {
  return stream ? as_stream(stream) : m->own_stream;
}

}  // namespace

// ======================================================================
// C ABI
// ======================================================================

namespace bmx {

// Allocates a model of shape cfg with uninitialised weights and the forward
// workspace for up to max_tokens tokens; the caller fills the weights.
int qwen3_alloc(const bmx_qwen3_config* cfg, int max_tokens, bmx_qwen3** out) {
  if (!cfg || !out) return set_error(BMX_E_ARG, "qwen3_create: null pointer");
  *out = nullptr;
  if (cfg->bits != 4 || cfg->group_size != 64)
    return set_error(BMX_E_UNSUPPORTED, "qwen3_create: only bits=4, group_size=64 (got %d, %d)", cfg->bits,
                     cfg->group_size);
  if (cfg->head_dim != 128 || cfg->n_kv_heads <= 0 || cfg->n_heads % cfg->n_kv_heads || cfg->hidden % 64 ||
      cfg->inter % 64 || (cfg->n_heads * cfg->head_dim) % 64 || cfg->layers <= 0 || cfg->vocab <= 0)
    return set_error(BMX_E_SHAPE, "qwen3_create: unsupported shape");
  if (max_tokens < 1 || max_tokens > 65535) return set_error(BMX_E_ARG, "qwen3_create: max_tokens=%d", max_tokens);
  bmx_qwen3* m = new bmx_qwen3();
  m->cfg = *cfg;
  m->max_tokens = max_tokens;
  m->rope = make_rope_table(cfg->head_dim, cfg->rope_theta);
  const int H = cfg->hidden, I = cfg->inter, qd = cfg->n_heads * cfg->head_dim, kvd = cfg->n_kv_heads * cfg->head_dim;
  hipStream_t st = nullptr;
  int rc = alloc_qlin(m, &m->embed, cfg->vocab, H);
  if (!rc && !cfg->tied) rc = alloc_qlin(m, &m->lm_head, cfg->vocab, H);
  if (!rc) rc = dalloc_t(m, &m->final_norm, static_cast<size_t>(H));
  m->layers.resize(cfg->layers);
  const int dims[NSLOT][2] = {{qd, H}, {kvd, H}, {kvd, H}, {H, qd}, {I, H}, {I, H}, {H, I}};
  for (int l = 0; !rc && l < cfg->layers; l++) {
    Layer& L = m->layers[l];
    for (int sl = 0; !rc && sl < NSLOT; sl++) rc = alloc_qlin(m, &L.p[sl], dims[sl][0], dims[sl][1], true);
    if (!rc) rc = dalloc_t(m, &L.in_norm, static_cast<size_t>(H));
    if (!rc) rc = dalloc_t(m, &L.post_norm, static_cast<size_t>(H));
    if (!rc) rc = dalloc_t(m, &L.q_norm, static_cast<size_t>(cfg->head_dim));
    if (!rc) rc = dalloc_t(m, &L.k_norm, static_cast<size_t>(cfg->head_dim));
  }
  // workspace
  const size_t T = static_cast<size_t>(max_tokens);
  if (!rc) rc = dalloc_t(m, &m->x, T * H);
  if (!rc) rc = dalloc_t(m, &m->h, T * H);
  if (!rc) rc = dalloc_t(m, &m->q, T * qd);
  if (!rc) rc = dalloc_t(m, &m->k, T * kvd);
  if (!rc) rc = dalloc_t(m, &m->v, T * kvd);
  if (!rc) rc = dalloc_t(m, &m->qr, T * qd);
  if (!rc) rc = dalloc_t(m, &m->rope_cs, T * 64);
  if (!rc) rc = dalloc_t(m, &m->att, T * qd);
  if (!rc) rc = dalloc_t(m, &m->o, T * H);
  if (!rc) rc = dalloc_t(m, &m->g, T * I);
  if (!rc) rc = dalloc_t(m, &m->u, T * I);
  if (!rc) rc = dalloc_t(m, &m->a, T * I);
  if (!rc) rc = dalloc_t(m, &m->logits1, static_cast<size_t>(cfg->vocab));
  if (!rc) rc = dalloc_t(m, &m->vlogits, static_cast<size_t>(kMaxSpecK) * cfg->vocab);
  // attention split partials: 256 splits of 256 keys (65536 cached
  // positions) for every forward of up to 16 tokens, so that a verify row
  // takes the split-key path exactly where a decode step does and the two
  // stay bit-identical at any context a decode step covers (Hq * 16 * 256
  // * 130 floats: 68 MB at 32 query heads)
  m->attn_ws_floats = attention_workspace_floats(cfg->n_heads, 16, 256);
  if (!rc) rc = dalloc_t(m, &m->attn_ws, m->attn_ws_floats);
  // the arrival counters at its head start at zero (and every call leaves them so)
  if (!rc) rc = check_hip(hipMemsetAsync(m->attn_ws, 0, m->attn_ws_floats * sizeof(float), st), "hipMemsetAsync");
  if (!rc) attention_prepare(st);
  for (int sl = 0; sl < NSLOT; sl++)
    m->qmm_ws_floats = std::max(m->qmm_ws_floats, qmm_workspace_floats(max_tokens, dims[sl][0], dims[sl][1]));
  m->qmm_ws_floats = std::max(m->qmm_ws_floats, qmm_workspace_floats(max_tokens, cfg->vocab, H));
  // the o and down GEMVs of up to 8 tokens may split K (matrix-core GEMV)
  m->qmm_ws_floats = std::max(m->qmm_ws_floats, qmvx_workspace_floats(8, H, cfg->n_heads * cfg->head_dim));
  m->qmm_ws_floats = std::max(m->qmm_ws_floats, qmvx_workspace_floats(8, H, cfg->inter));
  if (!rc && m->qmm_ws_floats) rc = dalloc_t(m, &m->qmm_ws, m->qmm_ws_floats);
  if (!rc) rc = dalloc_t(m, &m->ids, T);
  if (!rc) rc = dalloc_t(m, &m->tok_u, T < 64 ? 64 : T);
  if (!rc) rc = dalloc_t(m, &m->next_tok, 64);
  if (!rc) rc = dalloc_t(m, &m->step_io, 4);
  m->amax_cap = cfg->vocab / 4 + 64;  // workgroups of the lm_head GEMV (>= 4 rows each)
  if (!rc) rc = dalloc_t(m, &m->amax, static_cast<size_t>(m->amax_cap));
  if (!rc) rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&m->host_tok), 64 * sizeof(uint32_t), hipHostMallocDefault), "hipHostMalloc");
  if (!rc) rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&m->host_stage), T * sizeof(uint32_t), hipHostMallocDefault), "hipHostMalloc");
  if (!rc)
    rc = check_hip(hipHostMalloc(reinterpret_cast<void**>(&m->ring), kRing * sizeof(uint32_t),
                                 hipHostMallocMapped | hipHostMallocCoherent),
                   "hipHostMalloc");
  if (!rc) rc = check_hip(hipHostGetDevicePointer(reinterpret_cast<void**>(&m->ring_dev), m->ring, 0), "ring address");
  if (!rc)
    for (int i = 0; i < kRing; i++) m->ring[i] = kRingEmpty;
  if (!rc) rc = check_hip(hipEventCreateWithFlags(&m->stage_done, hipEventDisableTiming), "event create");
  if (!rc) rc = check_hip(hipEventRecord(m->stage_done, st), "event record");
  if (!rc) rc = check_hip(hipStreamCreate(&m->own_stream), "stream create");
  if (!rc) rc = check_hip(hipStreamSynchronize(st), "init sync");
  if (rc) {
    bmx_qwen3_destroy(m);
    return rc;
  }
  *out = m;
  return BMX_OK;
}

// Every weight tensor of the model under its MLX checkpoint name, in the
// order Qwen3::load takes them (crates/base-mlx-core/src/model/qwen3.rs:
// 194-295; names via qlin / rms, qwen3.rs:585-605).
std::vector<WeightSlot> qwen3_weight_slots(bmx_qwen3* m) {
  const bmx_qwen3_config& c = m->cfg;
  std::vector<WeightSlot> v;
  auto qlin = [&](const std::string& prefix, const QLin& q) {
    v.push_back({prefix + ".weight", q.w, q.N, q.K / 8, true});
    v.push_back({prefix + ".scales", q.s, q.N, q.K / 64, false});
    v.push_back({prefix + ".biases", q.b, q.N, q.K / 64, false});
  };
  auto norm = [&](const std::string& name, uint16_t* p, int n) { v.push_back({name, p, 1, n, false}); };
  qlin("model.embed_tokens", m->embed);
  static const char* const kProj[NSLOT] = {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj",
                                           "self_attn.o_proj", "mlp.gate_proj",    "mlp.up_proj",
                                           "mlp.down_proj"};
  for (int l = 0; l < c.layers; l++) {
    const std::string p = "model.layers." + std::to_string(l) + ".";
    Layer& L = m->layers[l];
    norm(p + "input_layernorm.weight", L.in_norm, c.hidden);
    for (int sl = 0; sl < NSLOT; sl++) qlin(p + kProj[sl], L.p[sl]);
    norm(p + "self_attn.q_norm.weight", L.q_norm, c.head_dim);
    norm(p + "self_attn.k_norm.weight", L.k_norm, c.head_dim);
    norm(p + "post_attention_layernorm.weight", L.post_norm, c.hidden);
  }
  norm("model.norm.weight", m->final_norm, c.hidden);
  if (!c.tied) qlin("lm_head", m->lm_head);
  return v;
}

}  // namespace bmx

extern "C" int bmx_qwen3_create_random(const bmx_qwen3_config* cfg, uint64_t seed, double sigma, int max_tokens,
                                       bmx_qwen3** out) {
  bmx_qwen3* m = nullptr;
  if (int rc = qwen3_alloc(cfg, max_tokens, &m)) return rc;
  const int H = cfg->hidden;
  const float c = static_cast<float>(sigma / kIrwin4Std);
  hipStream_t st = nullptr;
  int rc = launch_init_qlinear(tensor_seed(seed, -1, 0), cfg->vocab, H, c, m->embed.w, m->embed.s, m->embed.b, st);
  if (!rc && !cfg->tied)
    rc = launch_init_qlinear(tensor_seed(seed, -2, 0), cfg->vocab, H, c, m->lm_head.w, m->lm_head.s, m->lm_head.b, st);
  if (!rc) rc = fill_ones(m->final_norm, H, st);
  for (int l = 0; !rc && l < cfg->layers; l++) {
    Layer& L = m->layers[l];
    for (int sl = 0; !rc && sl < NSLOT; sl++)
      rc = launch_init_qlinear(tensor_seed(seed, l, sl), L.p[sl].N, L.p[sl].K, c, L.p[sl].w, L.p[sl].s, L.p[sl].b, st);
    if (!rc) rc = fill_ones(L.in_norm, H, st);
    if (!rc) rc = fill_ones(L.post_norm, H, st);
    if (!rc) rc = fill_ones(L.q_norm, cfg->head_dim, st);
    if (!rc) rc = fill_ones(L.k_norm, cfg->head_dim, st);
  }
  if (!rc) rc = repack_prefill_weights(m, st);
  if (!rc) rc = check_hip(hipStreamSynchronize(st), "init sync");
  if (rc) {
    bmx_qwen3_destroy(m);
    return rc;
  }
  *out = m;
  return BMX_OK;
}

extern "C" void bmx_qwen3_destroy(bmx_qwen3* m) {
  if (!m) return;
  (void)hipDeviceSynchronize();
  drop_graph(m);
  for (void* p : m->allocs) (void)hipFree(p);
  if (m->host_tok) (void)hipHostFree(m->host_tok);
  if (m->host_stage) (void)hipHostFree(m->host_stage);
  if (m->ring) (void)hipHostFree(m->ring);
  if (m->stage_done) (void)hipEventDestroy(m->stage_done);
  if (m->own_stream) (void)hipStreamDestroy(m->own_stream);
  delete m;
}

extern "C" int bmx_qwen3_qlinear(bmx_qwen3* m, int layer, int slot, uint32_t** w, bmx_bf16** s, bmx_bf16** b, int* N,
                                 int* K) {
  if (!m || !w || !s || !b || !N || !K) return set_error(BMX_E_ARG, "qwen3_qlinear: null pointer");
  const QLin* q = nullptr;
  if (layer == -1) q = &m->embed;
  else if (layer == -2) q = &head_of(m);
  else if (layer >= 0 && layer < m->cfg.layers && slot >= 0 && slot < NSLOT) q = &m->layers[layer].p[slot];
  else return set_error(BMX_E_ARG, "qwen3_qlinear: layer %d slot %d", layer, slot);
  // the caller may write through these: the prefill GEMMs' group-major
  // copies are rewritten from them before the next GEMM reads them
  if (layer >= 0) m->gm_stale = true;
  *w = q->w;
  *s = q->s;
  *b = q->b;
  *N = q->N;
  *K = q->K;
  return BMX_OK;
}

extern "C" int bmx_kv_create(const bmx_qwen3* m, int capacity, bmx_kv_cache** out) {
  if (!m || !out) return set_error(BMX_E_ARG, "kv_create: null pointer");
  *out = nullptr;
  if (capacity <= 0) return set_error(BMX_E_ARG, "kv_create: capacity=%d", capacity);
  static std::atomic<uint64_t> next_id{1};
  bmx_kv_cache* c = new bmx_kv_cache();
  c->id = next_id.fetch_add(1);
  c->layers = m->cfg.layers;
  c->nkv = m->cfg.n_kv_heads;
  c->hd = m->cfg.head_dim;
  c->cap = capacity;
  const size_t n = static_cast<size_t>(c->layers) * 2 * c->nkv * capacity * c->hd;
  hipError_t e = hipMalloc(reinterpret_cast<void**>(&c->data), n * 2);
  if (e != hipSuccess) {
    delete c;
    return set_error(BMX_E_ALLOC, "kv_create: hipMalloc(%zu): %s", n * 2, hipGetErrorString(e));
  }
  // the reference seeds the cache from a zeros buffer (qwen3.rs:457-488)
  e = hipMemset(c->data, 0, n * 2);
  if (e != hipSuccess) {
    (void)hipFree(c->data);
    delete c;
    return check_hip(e, "kv_create: memset");
  }
  *out = c;
  return BMX_OK;
}

extern "C" void bmx_kv_destroy(bmx_kv_cache* c) {
  if (!c) return;
  (void)hipDeviceSynchronize();
  (void)hipFree(c->data);
  delete c;
}

extern "C" int bmx_kv_seq_len(const bmx_kv_cache* c) { return c ? c->seq_len : 0; }
extern "C" int bmx_kv_capacity(const bmx_kv_cache* c) { return c ? c->cap : 0; }
extern "C" void bmx_kv_reset(bmx_kv_cache* c) {
  if (c) c->seq_len = 0;
}
extern "C" void bmx_kv_truncate(bmx_kv_cache* c, int target) {
  if (!c || target >= c->seq_len) return;  // qwen3.rs:150-153
  c->seq_len = target < 0 ? 0 : target;
}
extern "C" bmx_bf16* bmx_kv_data(bmx_kv_cache* c) { return c ? c->data : nullptr; }

extern "C" int bmx_kv_fill_synthetic(bmx_kv_cache* c, uint64_t seed, int seq_len, void* stream) {
  if (!c) return set_error(BMX_E_ARG, "kv_fill_synthetic: null cache");
  if (seq_len < 0 || seq_len > c->cap) return set_error(BMX_E_KV_CAPACITY, "kv_fill_synthetic: %d > %d", seq_len, c->cap);
  if (int rc = launch_fill_kv_synthetic(c->data, static_cast<int64_t>(c->layers) * 2 * c->nkv, c->cap, c->hd, seq_len,
                                        seed, static_cast<float>(1.0 / kIrwin4Std), as_stream(stream)))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(as_stream(stream)), "kv fill sync")) return rc;
  c->seq_len = seq_len;
  return BMX_OK;
}

extern "C" int bmx_qwen3_forward(bmx_qwen3* m, bmx_kv_cache* c, const uint32_t* tokens, int M, int all_logits,
                                 bmx_bf16* logits, void* stream) {
  if (!m || !c || !tokens || !logits) return set_error(BMX_E_ARG, "qwen3_forward: null pointer");
  if (M <= 0) return set_error(BMX_E_ARG, "qwen3_forward: M=%d", M);
  if (M > m->max_tokens) return set_error(BMX_E_SHAPE, "qwen3_forward: M=%d > max_tokens %d", M, m->max_tokens);
  if (c->layers != m->cfg.layers || c->nkv != m->cfg.n_kv_heads)  // qwen3.rs:351-358
    return set_error(BMX_E_SHAPE, "cache layer count %d != model layers %d", c->layers, m->cfg.layers);
  if (c->seq_len + M > c->cap)  // qwen3.rs:423-428
    return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", c->seq_len + M, c->cap);
  hipStream_t st = pick_stream(m, stream);
  if (int rc = upload_tokens(m, tokens, M, st)) return rc;
  if (int rc = forward_device(m, c, M, c->seq_len, nullptr, all_logits != 0, logits, st)) return rc;
  c->seq_len += M;  // qwen3.rs:557
  return BMX_OK;
}

// One greedy decode step on device: token tok (host) at position seq_len,
// through the captured graph; the argmax lands in *next (host).
static int graph_step(bmx_qwen3* m, bmx_kv_cache* c, hipStream_t st, uint32_t tok, uint32_t* next) {
  if (c->seq_len + 1 > c->cap)
    return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", c->seq_len + 1, c->cap);
  if (int rc = ensure_graph(m, c, st)) return rc;
  m->host_tok[0] = tok;
  m->host_tok[1] = static_cast<uint32_t>(c->seq_len);
  m->host_tok[2] = 0;
  m->host_tok[3] = 0;  // ring count: this replay publishes to slot 0, whatever ran before
  if (int rc = check_hip(hipMemcpyAsync(m->step_io, &m->host_tok[0], 16, hipMemcpyHostToDevice, st), "set token"))
    return rc;
  if (int rc = check_hip(hipGraphLaunch(m->graph, st), "graph launch")) return rc;
  if (int rc = check_hip(hipMemcpyAsync(&m->host_tok[2], m->step_io + 2, 4, hipMemcpyDeviceToHost, st), "read token"))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(st), "decode sync")) return rc;
  c->seq_len += 1;
  *next = m->host_tok[2];
  return BMX_OK;
}

extern "C" int bmx_qwen3_decode_step(bmx_qwen3* m, bmx_kv_cache* c, uint32_t token, uint32_t* next_token,
                                     bmx_bf16* logits, void* stream) {
  if (!m || !c || !next_token) return set_error(BMX_E_ARG, "decode_step: null pointer");
  if (token >= static_cast<uint32_t>(m->cfg.vocab)) return set_error(BMX_E_ARG, "decode_step: token %u", token);
  hipStream_t st = pick_stream(m, stream);
  if (int rc = graph_step(m, c, st, token, next_token)) return rc;
  if (logits)
    return check_hip(hipMemcpy(logits, m->logits1, static_cast<size_t>(m->cfg.vocab) * 2, hipMemcpyDeviceToDevice),
                     "copy logits");
  return BMX_OK;
}

// Waits for the decode graph to publish ring slot `slot` (polling the mapped
// host memory), watching the stream so that a failed or drained stream ends
// the wait with an error instead of a hang.
static int ring_wait(bmx_qwen3* m, hipStream_t st, int slot, uint32_t* tok) {
  volatile uint32_t* r = m->ring + slot;
  for (unsigned spin = 1;; spin++) {
    const uint32_t v = *r;
    if (v != kRingEmpty) {
      *tok = v;
      return BMX_OK;
    }
    if ((spin & 255) == 0) {
      const hipError_t e = hipStreamQuery(st);
      if (e == hipSuccess) {
        // the stream is idle, so the slot's store has landed if it was made
        const uint32_t v2 = *r;
        if (v2 == kRingEmpty)
          return set_error(static_cast<int>(hipErrorUnknown), "decode: step %d ended without its token", slot);
        *tok = v2;
        return BMX_OK;
      }
      if (e != hipErrorNotReady) return check_hip(e, "decode wait");
    }
    __builtin_ia32_pause();
  }
}

// The greedy decode loop of engine.rs:103-115 from the token the prefill
// picked: emit `first` unless it is an eos token, then decode one token per
// step from the last one emitted until an eos token (not emitted) or
// max_new tokens.  The steps are graph replays queued up to kAhead ahead of
// the token being checked: each replay takes its token and position from
// the previous one on the device and publishes its token to the host ring,
// so the GPU runs step after step while the host checks tokens behind it.
// When an eos token ends the loop, the replays queued past it are drained
// and the cache is rewound to the steps the loop took (their K/V rows lie at
// and beyond seq_len, where the next step writes before any step reads).
// Output, seq_len and errors are those of one synchronous step at a time,
// including the capacity error at the step that would not fit.
static int decode_loop(bmx_qwen3* m, bmx_kv_cache* c, hipStream_t st, uint32_t first, int max_new,
                       const uint32_t* eos, int n_eos, uint32_t* out, int* n_out) {
  int n = 0;
  *n_out = 0;
  if (is_eos(first, eos, n_eos)) return BMX_OK;
  out[n++] = first;
  const int steps = max_new - 1;                         // steps the loop takes without an eos
  const int fit = std::min(steps, c->cap - c->seq_len);  // of which the cache holds
  const int seq0 = c->seq_len;
  int rc = BMX_OK, launched = 0, done = 0;
  if (fit > 0) {
    rc = ensure_graph(m, c, st);
    if (!rc) {
      m->host_tok[0] = first;
      m->host_tok[1] = static_cast<uint32_t>(seq0);
      m->host_tok[2] = 0;
      m->host_tok[3] = 0;  // ring count: step i publishes to slot i
      rc = check_hip(hipMemcpyAsync(m->step_io, &m->host_tok[0], 16, hipMemcpyHostToDevice, st), "set token");
    }
  }
  while (!rc && done < steps) {
    while (launched < fit && launched - done < kAhead) {
      m->ring[launched & (kRing - 1)] = kRingEmpty;
      rc = check_hip(hipGraphLaunch(m->graph, st), "graph launch");
      if (rc) break;
      launched++;
    }
    if (rc) break;
    if (done == fit) {
      rc = set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", seq0 + fit + 1, c->cap);
      break;
    }
    uint32_t t;
    rc = ring_wait(m, st, done & (kRing - 1), &t);
    if (rc) break;
    done++;
    if (is_eos(t, eos, n_eos)) break;
    out[n++] = t;
  }
  // the replays queued past an eos, and the staging copy, finish here
  const int rs = check_hip(hipStreamSynchronize(st), "decode sync");
  c->seq_len = seq0 + done;
  *n_out = n;
  return rc ? rc : rs;
}

extern "C" int bmx_decode_greedy(bmx_qwen3* m, bmx_kv_cache* c, uint32_t token, int max_new, const uint32_t* eos,
                                 int n_eos, uint32_t* out, int* n_out, void* stream) {
  if (!m || !c || !out || !n_out || (n_eos > 0 && !eos)) return set_error(BMX_E_ARG, "decode: null pointer");
  *n_out = 0;
  if (max_new <= 0) return set_error(BMX_E_ARG, "decode: max_new=%d", max_new);
  if (token >= static_cast<uint32_t>(m->cfg.vocab)) return set_error(BMX_E_ARG, "decode: token %u", token);
  if (c->layers != m->cfg.layers || c->nkv != m->cfg.n_kv_heads)  // qwen3.rs:351-358
    return set_error(BMX_E_SHAPE, "cache layer count %d != model layers %d", c->layers, m->cfg.layers);
  return decode_loop(m, c, pick_stream(m, stream), token, max_new, eos, n_eos, out, n_out);
}

extern "C" int bmx_generate_greedy(bmx_qwen3* m, bmx_kv_cache* c, const uint32_t* prompt, int P, int max_new,
                                   const uint32_t* eos, int n_eos, uint32_t* out, int* n_out, void* stream) {
  if (!m || !c || !prompt || !out || !n_out || (n_eos > 0 && !eos)) return set_error(BMX_E_ARG, "generate: null pointer");
  *n_out = 0;
  if (P <= 0 || max_new <= 0) return set_error(BMX_E_ARG, "generate: P=%d max_new=%d", P, max_new);
  hipStream_t st = pick_stream(m, stream);
  // prefill in chunks of max_tokens (a single forward in the reference,
  // engine.rs:98; chunking changes no result: every op is row-wise or
  // causal over the cache)
  int done = 0;
  while (done < P) {
    const int mm = std::min(P - done, m->max_tokens);
    const bool last = done + mm == P;
    if (c->seq_len + mm > c->cap)
      return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", c->seq_len + mm, c->cap);
    if (int rc = upload_tokens(m, prompt + done, mm, st)) return rc;
    if (int rc = forward_device(m, c, mm, c->seq_len, nullptr, false, m->logits1, st)) return rc;
    c->seq_len += mm;
    done += mm;
    if (last) {
      if (int rc = launch_argmax(m->logits1, 1, m->cfg.vocab, m->next_tok, st)) return rc;
    }
  }
  if (int rc = check_hip(hipMemcpyAsync(&m->host_tok[2], m->next_tok, 4, hipMemcpyDeviceToHost, st), "read token"))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(st), "prefill sync")) return rc;
  return decode_loop(m, c, st, m->host_tok[2], max_new, eos, n_eos, out, n_out);
}

// Verify forward for the speculative loop: tokens (host) -> argmax of every
// row (host).
static int forward_argmax(bmx_qwen3* m, bmx_kv_cache* c, const uint32_t* toks, int M, bool all, uint32_t* preds,
                          uint16_t* logits, hipStream_t st) {
  if (c->seq_len + M > c->cap)
    return set_error(BMX_E_KV_CAPACITY, "KV cache exhausted: requested %d positions, max %d", c->seq_len + M, c->cap);
  if (int rc = upload_tokens(m, toks, M, st)) return rc;
  if (int rc = forward_device(m, c, M, c->seq_len, nullptr, all, logits, st)) return rc;
  c->seq_len += M;
  const int rows = all ? M : 1;
  if (int rc = launch_argmax(logits, rows, m->cfg.vocab, m->next_tok, st)) return rc;
  if (int rc = check_hip(hipMemcpyAsync(&m->host_tok[8], m->next_tok, rows * 4, hipMemcpyDeviceToHost, st), "read preds"))
    return rc;
  if (int rc = check_hip(hipStreamSynchronize(st), "verify sync")) return rc;
  memcpy(preds, &m->host_tok[8], rows * 4);
  return BMX_OK;
}

extern "C" int bmx_speculative_generate(bmx_qwen3* target, bmx_kv_cache* tc, bmx_qwen3* draft, bmx_kv_cache* dc,
                                        const uint32_t* prompt, int P, int max_new, int spec_k, const uint32_t* eos,
                                        int n_eos, uint32_t* out, int* n_out, int64_t* stats, void* stream) {
  if (!target || !tc || !draft || !dc || !prompt || !out || !n_out || (n_eos > 0 && !eos))
    return set_error(BMX_E_ARG, "speculative: null pointer");
  *n_out = 0;
  if (draft->cfg.vocab != target->cfg.vocab)  // check_compatible, speculative.rs:40-54
    return set_error(BMX_E_ARG, "draft/target vocab mismatch: target=%d draft=%d", target->cfg.vocab, draft->cfg.vocab);
  if (P <= 0 || max_new <= 0) return set_error(BMX_E_ARG, "speculative: P=%d max_new=%d", P, max_new);
  if (spec_k < 2 || spec_k > kMaxSpecK)
    return set_error(BMX_E_ARG, "speculative: spec_k=%d outside 2..%d", spec_k, kMaxSpecK);
  if (spec_k > target->max_tokens) return set_error(BMX_E_SHAPE, "speculative: spec_k > target max_tokens");
  // the caches may already hold context (a continued conversation): every
  // rewind below is relative to where each one starts
  const int t0 = tc->seq_len, d0 = dc->seq_len;
  hipStream_t st = pick_stream(target, stream);
  int64_t iters = 0, proposed = 0, accepted = 0;
  int n = 0, rc = BMX_OK;
  uint32_t leader = 0, dnext = 0;
  uint16_t* const tlog = target->vlogits;  // the verify rows' logits: [spec_k, vocab]
  // prefill both (speculative.rs:75-79): only the target's last row is used
  // and the draft's logits are discarded, so only those rows are computed
  {
    int done = 0;
    while (!rc && done < P) {
      const int mm = std::min(P - done, target->max_tokens);
      uint32_t pr;
      rc = forward_argmax(target, tc, prompt + done, mm, false, &pr, target->logits1, st);
      leader = pr;
      done += mm;
    }
    done = 0;
    while (!rc && done < P) {
      const int mm = std::min(P - done, draft->max_tokens);
      uint32_t pr;
      rc = forward_argmax(draft, dc, prompt + done, mm, false, &pr, draft->logits1, st);
      done += mm;
    }
  }
  if (rc || is_eos(leader, eos, n_eos)) goto done;
  out[n++] = leader;
  if ((rc = graph_step(draft, dc, st, leader, &dnext))) goto done;  // :104
  while (n < max_new) {
    uint32_t drafts[8], vin[8], preds[8];
    int nd = 0;
    for (int i = 0; i < spec_k - 1; i++) {  // :124-137
      const uint32_t d = dnext;
      drafts[nd++] = d;
      if ((rc = graph_step(draft, dc, st, d, &dnext))) goto done;
      if (is_eos(d, eos, n_eos)) break;
    }
    vin[0] = leader;
    for (int i = 0; i < nd; i++) vin[i + 1] = drafts[i];
    if ((rc = forward_argmax(target, tc, vin, nd + 1, true, preds, tlog, st))) goto done;  // :146-173
    proposed += nd;
    iters++;
    int na = 0;
    uint32_t bonus = preds[nd];
    for (int i = 0; i < nd; i++) {  // :175-192
      if (preds[i] == drafts[i]) na++;
      else {
        bonus = preds[i];
        break;
      }
    }
    accepted += na;
    bool stop = false;
    for (int i = 0; i < na; i++) {  // :201-211
      if (n >= max_new || is_eos(drafts[i], eos, n_eos)) {
        stop = true;
        break;
      }
      out[n++] = drafts[i];
    }
    if (stop || n >= max_new || is_eos(bonus, eos, n_eos)) break;
    out[n++] = bonus;
    // rewind both caches to prompt + emitted - 1 (:227, :234), keeping the buffers
    bmx_kv_truncate(tc, t0 + P + n - 1);
    bmx_kv_truncate(dc, d0 + P + n - 1);
    leader = bonus;
    if ((rc = graph_step(draft, dc, st, leader, &dnext))) goto done;  // :238-239
  }
done:
  *n_out = n;
  if (stats) {
    stats[0] = iters;
    stats[1] = proposed;
    stats[2] = accepted;
  }
  return rc;
}
