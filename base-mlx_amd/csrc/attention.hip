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
// Decomposition (flash-decoding).  A workgroup of W waves owns one kv head,
// a tile of TQ query tokens (R = TQ * Hq/Hkv query rows, all sharing the kv
// head) and one of NS splits of the key range.  It walks its split in chunks
// of 64*W keys with an online softmax:
//   QK: lane = key; the key row (128 bf16) sits in registers, query rows
//       (pre-scaled, fp32) are broadcast from LDS;
//   softmax: one wave per row updates the running max / sum;
//   PV: thread = (row, pair of dims); V rows are read coalesced, p from LDS.
// With NS > 1 the unnormalised partial (o, m, l) goes to a workspace and a
// combine kernel merges the splits.
#include <math.h>

#include "bmx_device.h"

namespace bmx {
namespace {

constexpr int kD = 128;  // head_dim

struct AttnParams {
  const uint16_t* q;  // [Hq, M, 128]
  const uint16_t* k;  // [Hkv, cap, 128]
  const uint16_t* v;  // [Hkv, cap, 128]
  uint16_t* out;      // [M, Hq*128]
  float* part_o;      // [Hq, M, NS, 128]
  float* part_ml;     // [Hq, M, NS, 2]
  const int* offset_dev;
  int offset;
  int Hq, Hkv, M, cap;
  int tq;     // query tokens per workgroup
  int ns;     // key splits
  int causal;
  float scale;
};

template <int W, int IT>
__global__ void __launch_bounds__(W * 64) attn_kernel(const AttnParams p) {
  constexpr int CH = 64 * W;  // keys per chunk
  extern __shared__ __align__(16) unsigned char smem[];
  const int rep = p.Hq / p.Hkv;
  const int kvh = blockIdx.x;
  const int qt = blockIdx.y;
  const int split = blockIdx.z;
  const int t0 = qt * p.tq;
  const int tn = min(p.tq, p.M - t0);
  const int R = tn * rep;  // rows: r = j * tn + i  (head kvh*rep + j, token t0 + i)
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int offset = p.offset_dev ? *p.offset_dev : p.offset;
  const int L = offset + p.M;  // keys in the cache view
  // keys this tile can see: causal -> up to offset + t0 + tn - 1
  const int Lt = p.causal ? offset + t0 + tn : L;
  const int per = ((Lt + p.ns - 1) / p.ns + CH - 1) / CH * CH;
  const int kbeg = split * per;
  const int kend = min(Lt, kbeg + per);

  float* qs = reinterpret_cast<float*>(smem);  // [R][128]
  float* ps = qs + R * kD;                     // [R][CH]
  float* st = ps + R * CH;                     // [R][3]: m, l, alpha

  for (int e = threadIdx.x; e < R * kD; e += W * 64) {
    const int r = e / kD, d = e - r * kD;
    const int j = r / tn, i = r - j * tn;
    qs[e] = bf2f(p.q[(static_cast<int64_t>(kvh * rep + j) * p.M + t0 + i) * kD + d]) * p.scale;
  }
  for (int r = threadIdx.x; r < R; r += W * 64) {
    st[r * 3 + 0] = -INFINITY;
    st[r * 3 + 1] = 0.0f;
  }
  // PV accumulators: thread owns dims (2*lane, 2*lane+1) of rows wave + W*it
  float acc[IT][2];
#pragma unroll
  for (int it = 0; it < IT; it++) acc[it][0] = acc[it][1] = 0.0f;
  __syncthreads();

  const uint16_t* kb = p.k + static_cast<int64_t>(kvh) * p.cap * kD;
  const uint16_t* vb = p.v + static_cast<int64_t>(kvh) * p.cap * kD;
  for (int c0 = kbeg; c0 < kend; c0 += CH) {
    // ---- QK: lane = key ----
    {
      const int j = c0 + wave * 64 + lane;
      const bool kok = j < kend;
      uint4 kr[16];
      const uint4* kp = reinterpret_cast<const uint4*>(kb + static_cast<int64_t>(kok ? j : c0) * kD);
#pragma unroll
      for (int c = 0; c < 16; c++) kr[c] = kp[c];
      for (int r = 0; r < R; r++) {
        const float* qr = qs + r * kD;
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < 16; c++) {
          const uint32_t w4[4] = {kr[c].x, kr[c].y, kr[c].z, kr[c].w};
          const float4 qa = *reinterpret_cast<const float4*>(qr + c * 8);
          const float4 qb = *reinterpret_cast<const float4*>(qr + c * 8 + 4);
          s += qa.x * bf2f(w4[0] & 0xffffu) + qa.y * bf2f(w4[0] >> 16) + qa.z * bf2f(w4[1] & 0xffffu) +
               qa.w * bf2f(w4[1] >> 16) + qb.x * bf2f(w4[2] & 0xffffu) + qb.y * bf2f(w4[2] >> 16) +
               qb.z * bf2f(w4[3] & 0xffffu) + qb.w * bf2f(w4[3] >> 16);
        }
        const int t = t0 + (r % tn);
        const bool vis = kok && (!p.causal || j <= offset + t);
        ps[r * CH + wave * 64 + lane] = vis ? s : -INFINITY;
      }
    }
    __syncthreads();
    // ---- online softmax: one wave per row ----
    for (int r = wave; r < R; r += W) {
      float* pr = ps + r * CH;
      float mx = -INFINITY;
      for (int c = lane; c < CH; c += 64) mx = fmaxf(mx, pr[c]);
      for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, 64));
      const float m_old = st[r * 3 + 0];
      const float m_new = fmaxf(m_old, mx);
      float sum = 0.0f;
      for (int c = lane; c < CH; c += 64) {
        const float e = (m_new == -INFINITY) ? 0.0f : expf(pr[c] - m_new);
        pr[c] = e;
        sum += e;
      }
      sum = wave_sum_xor(sum, 64);
      if (lane == 0) {
        const float alpha = (m_old == -INFINITY) ? 0.0f : expf(m_old - m_new);
        st[r * 3 + 0] = m_new;
        st[r * 3 + 1] = st[r * 3 + 1] * alpha + sum;
        st[r * 3 + 2] = alpha;
      }
    }
    __syncthreads();
    // ---- PV: thread = (row wave + W*it, dims 2*lane .. 2*lane+1) ----
    {
      const int nk = min(CH, kend - c0);
#pragma unroll
      for (int it = 0; it < IT; it++) {
        const int r = wave + W * it;
        if (r < R) {
          const float alpha = st[r * 3 + 2];
          acc[it][0] *= alpha;
          acc[it][1] *= alpha;
        }
      }
      for (int c = 0; c < nk; c++) {
        const uint32_t vv = *reinterpret_cast<const uint32_t*>(vb + static_cast<int64_t>(c0 + c) * kD + 2 * lane);
        const float v0 = bf2f(vv & 0xffffu), v1 = bf2f(vv >> 16);
#pragma unroll
        for (int it = 0; it < IT; it++) {
          const int r = wave + W * it;
          if (r < R) {
            const float pv = ps[r * CH + c];
            acc[it][0] += pv * v0;
            acc[it][1] += pv * v1;
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- write ----
#pragma unroll
  for (int it = 0; it < IT; it++) {
    const int r = wave + W * it;
    if (r >= R) continue;
    const int j = r / tn, i = r - j * tn;
    const int h = kvh * rep + j, t = t0 + i;
    const float m = st[r * 3 + 0], l = st[r * 3 + 1];
    if (p.ns == 1) {
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      uint16_t* o = p.out + static_cast<int64_t>(t) * p.Hq * kD + h * kD + 2 * lane;
      o[0] = f2bf(acc[it][0] * inv);
      o[1] = f2bf(acc[it][1] * inv);
    } else {
      const int64_t base = (static_cast<int64_t>(h) * p.M + t) * p.ns + split;
      float* o = p.part_o + base * kD + 2 * lane;
      o[0] = acc[it][0];
      o[1] = acc[it][1];
      if (lane == 0) {
        p.part_ml[base * 2 + 0] = m;
        p.part_ml[base * 2 + 1] = l;
      }
    }
  }
}

// merge NS partials of each (head, token); one wave per pair
__global__ void __launch_bounds__(256) attn_combine_kernel(const AttnParams p) {
  const int wid = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (wid >= p.Hq * p.M) return;
  const int h = wid / p.M, t = wid - h * p.M;
  const int64_t base = static_cast<int64_t>(wid) * p.ns;
  float mx = -INFINITY;
  for (int s = 0; s < p.ns; s++) mx = fmaxf(mx, p.part_ml[(base + s) * 2]);
  float l = 0.0f, o0 = 0.0f, o1 = 0.0f;
  for (int s = 0; s < p.ns; s++) {
    const float m = p.part_ml[(base + s) * 2];
    if (m == -INFINITY) continue;
    const float w = expf(m - mx);
    l += w * p.part_ml[(base + s) * 2 + 1];
    o0 += w * p.part_o[(base + s) * kD + 2 * lane];
    o1 += w * p.part_o[(base + s) * kD + 2 * lane + 1];
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  uint16_t* o = p.out + static_cast<int64_t>(t) * p.Hq * kD + h * kD + 2 * lane;
  o[0] = f2bf(o0 * inv);
  o[1] = f2bf(o1 * inv);
}

template <int W>
int launch_w(const AttnParams& p, dim3 grid, int R, hipStream_t st) {
  const size_t lds = static_cast<size_t>(R) * (kD + 64 * W + 3) * 4;
  const int it = (R + W - 1) / W;
  if (R > 32 || R < 1) return set_error(BMX_E_SHAPE, "attention: %d query rows per workgroup", R);
  if (it <= 1) hipLaunchKernelGGL((attn_kernel<W, 1>), grid, dim3(W * 64), lds, st, p);
  else if (it <= 2) hipLaunchKernelGGL((attn_kernel<W, 2>), grid, dim3(W * 64), lds, st, p);
  else if (it <= 4) hipLaunchKernelGGL((attn_kernel<W, 4>), grid, dim3(W * 64), lds, st, p);
  else hipLaunchKernelGGL((attn_kernel<W, 8>), grid, dim3(W * 64), lds, st, p);
  return check_launch("attention");
}

}  // namespace

// Workspace floats needed for the split partials of one call.
size_t attention_workspace_floats(int Hq, int M, int ns) {
  return static_cast<size_t>(Hq) * M * ns * (kD + 2);
}

// Picks the query tile / split shape.  `max_ns` bounds the splits by the
// workspace available (0 = no workspace: single split).
void attention_shape(int Hq, int Hkv, int M, int L_max, int max_ns, int* tq, int* ns, int* w) {
  const int rep = Hq / Hkv;
  // R = tq * rep query rows share a workgroup; R <= 32 keeps LDS <= 50 KB
  *tq = M <= 8 ? M : 8;
  while (*tq > 1 && *tq * rep > 32) (*tq)--;
  *w = 4;
  const int qtiles = (M + *tq - 1) / *tq;
  const int blocks = Hkv * qtiles;
  int n = 1;
  const int chunks = (L_max + 64 * *w - 1) / (64 * *w);
  while (blocks * n < 512 && n * 2 <= chunks) n *= 2;
  if (n > max_ns) n = max_ns > 0 ? max_ns : 1;
  *ns = n;
}

int launch_attention(const uint16_t* q, const uint16_t* k, const uint16_t* v, uint16_t* out, float* ws,
                     size_t ws_floats, int Hq, int Hkv, int M, int D, int cap, int offset, const int* offset_dev,
                     int L_max, float scale, hipStream_t stream) {
  if (D != kD) return set_error(BMX_E_UNSUPPORTED, "attention: head_dim must be 128 (got %d)", D);
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv || M <= 0) return set_error(BMX_E_SHAPE, "attention: bad head counts");
  if (!offset_dev && (offset < 0 || offset + M > cap))
    return set_error(BMX_E_KV_CAPACITY, "attention: %d positions exceed capacity %d", offset + M, cap);
  int tq, ns, w;
  const int max_ns = ws ? static_cast<int>(ws_floats / (static_cast<size_t>(Hq) * M * (kD + 2))) : 1;
  attention_shape(Hq, Hkv, M, L_max, max_ns, &tq, &ns, &w);
  AttnParams p{q, k, v, out, ws, ws ? ws + static_cast<size_t>(Hq) * M * ns * kD : nullptr, offset_dev, offset,
               Hq, Hkv, M, cap, tq, ns, M > 1 ? 1 : 0, scale};
  const int rep = Hq / Hkv;
  const dim3 grid(Hkv, (M + tq - 1) / tq, ns);
  if (int rc = launch_w<4>(p, grid, tq * rep, stream)) return rc;
  if (ns > 1) {
    hipLaunchKernelGGL(attn_combine_kernel, dim3((Hq * M + 3) / 4), dim3(256), 0, stream, p);
    return check_launch("attention_combine");
  }
  return BMX_OK;
}

}  // namespace bmx

using namespace bmx;

extern "C" size_t bmx_attention_workspace_bytes(int n_heads, int M) {
  // splits are bounded by 64 for any call
  return attention_workspace_floats(n_heads, M, 64) * sizeof(float);
}

extern "C" int bmx_attention_gqa(const bmx_bf16* q, const bmx_bf16* k_cache, const bmx_bf16* v_cache, bmx_bf16* out,
                                 int n_heads, int n_kv_heads, int M, int head_dim, int capacity, int offset,
                                 float scale, void* workspace, size_t workspace_bytes, void* stream) {
  if (!q || !k_cache || !v_cache || !out) return set_error(BMX_E_ARG, "attention: null pointer");
  return launch_attention(q, k_cache, v_cache, out, static_cast<float*>(workspace), workspace_bytes / sizeof(float),
                          n_heads, n_kv_heads, M, head_dim, capacity, offset, nullptr, offset + M, scale,
                          as_stream(stream));
}
