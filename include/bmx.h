/*
 * bmx.h -- C ABI of the MI355X-native (gfx950) implementation of
 * base-mlx's 4-bit affine quantized matmul path (MLX format: uint32-packed
 * nibbles, group_size 64, bf16 per-group scales and biases) and the ops of
 * a Qwen3 decode step around it.
 *
 * Conventions (every entry point):
 *  - All tensor pointers are DEVICE pointers owned by the caller, row-major
 *    and contiguous unless a stride is given.  bf16 tensors are passed as
 *    raw 16-bit patterns (bmx_bf16).
 *  - `stream` is a hipStream_t (NULL = the default stream).  Calls enqueue
 *    work and return without synchronising.
 *  - Return value: 0 on success, a negative BMX_E_* code for an argument or
 *    shape error (nothing is enqueued), or a positive hipError_t.  The text
 *    for the last failure on the calling thread is bmx_last_error().  This
 *    mirrors mlx-c's `int` return, so a wrapper written like the reference's
 *    mlx_ext::slice_update (crates/base-mlx-core/src/mlx_ext.rs:58-61) maps
 *    rc != 0 to Error::Inference(String) unchanged.
 *  - No call aborts.  Calls are thread-compatible, not thread-safe per
 *    stream, like the reference's single-threaded model use
 *    (crates/base-mlx-server/src/state.rs:1-19).
 */
#ifndef BMX_H
#define BMX_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef uint16_t bmx_bf16;

#define BMX_OK 0
#define BMX_E_ARG (-1)         /* null pointer or invalid argument */
#define BMX_E_SHAPE (-2)       /* shape / size mismatch */
#define BMX_E_UNSUPPORTED (-3) /* bits != 4 or group_size != 64 */
#define BMX_E_KV_CAPACITY (-4) /* offset + M exceeds the KV capacity */
#define BMX_E_ALLOC (-5)       /* device allocation failed */
#define BMX_E_ALIGN (-6)       /* pointer alignment requirement not met */

/* Text of the last failure on this thread ("" if none). */
const char *bmx_last_error(void);
/* ABI version: (major << 16) | minor. */
int bmx_abi_version(void);

/* ------------------------------------------------------------------ */
/* Quantized matmul                                                    */
/* ------------------------------------------------------------------ */

/* y[M,N] = x[M,K] . dequant(w, scales, biases)^T   (transpose != 0)
 * w: [N, K*bits/32] uint32; scales, biases: [N, K/group_size] bf16;
 * x, y bf16; fp32 accumulation.  bits must be 4 and group_size 64;
 * transpose = 0 (W stored [K, N]) is BMX_E_UNSUPPORTED -- every call of the
 * reference passes true.  M <= 8 runs the streaming GEMV (qmv: dot2 on
 * the VALU, or the matrix cores when N and K are both >= 5120 -- chosen by
 * the shape alone, so a row's result never depends on M); larger M the
 * MFMA GEMM (qmm).  x and w must be 16-byte aligned.
 * Shapes that split K over workgroups (small GEMM grids; matrix-core GEMVs
 * with K >= 8192) keep fp32 partials in a device buffer the library owns
 * per (device, stream), allocated or grown on first use of a larger shape
 * on that stream (which synchronizes the stream): the first call of a
 * shape on a stream must not be inside graph capture.  Callers that must
 * not allocate use bmx_qmatmul_affine_ws.
 * Replaces: mlx_rs::ops::quantized_matmul(x, w, scales, biases, transpose,
 *   group_size, bits) -- mlx-c's mlx_quantized_matmul(res, x, w, scales,
 *   biases, transpose, group_size, bits, stream) -- as called by
 *   QLinear::forward (crates/base-mlx-core/src/model/qwen3.rs:30-41),
 *   QEmbedding::lm_head (qwen3.rs:80-91) and qkv_block / mlp_block
 *   (crates/base-mlx-core/src/model/kernels.rs:42-44, 69-75). */
int bmx_qmatmul_affine(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales,
                       const bmx_bf16 *biases, bmx_bf16 *y, int64_t M, int64_t N, int64_t K,
                       int transpose, int group_size, int bits, void *stream);

/* Bytes of split-K workspace bmx_qmatmul_affine_ws needs for an M x N x K
 * call (0: the shape does not split K, any workspace or NULL will do).
 * Host only.
 * Replaces: nothing in the reference (MLX sizes its temporaries itself);
 *   the companion of bmx_qmatmul_affine_ws. */
size_t bmx_qmatmul_workspace_bytes(int64_t M, int64_t N, int64_t K);

/* bmx_qmatmul_affine with the split-K partials in the caller's workspace
 * (device memory, 16-byte aligned, at least bmx_qmatmul_workspace_bytes(M,
 * N, K) bytes, else BMX_E_ARG and nothing enqueued).  It never allocates or
 * synchronizes, so it may be captured into a graph on any call.  Calls that
 * share a workspace must not run concurrently.
 * Replaces: the same quantized_matmul calls as bmx_qmatmul_affine
 *   (crates/base-mlx-core/src/model/qwen3.rs:30-41, 80-91). */
int bmx_qmatmul_affine_ws(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales,
                          const bmx_bf16 *biases, bmx_bf16 *y, int64_t M, int64_t N, int64_t K,
                          int transpose, int group_size, int bits, void *workspace, size_t workspace_bytes,
                          void *stream);

/* bmx_qmatmul_affine with the split-K partials in a scratch array of the
 * library's own (a file-scope device array of 16 MiB that each GPU the
 * library runs on holds until the process ends): no allocation, no caller
 * workspace, no synchronization.  A shape whose partials need more than
 * 16 MiB (bmx_qmatmul_workspace_bytes) is BMX_E_SHAPE.  All calls on one
 * GPU share the array, so calls that overlap on one GPU (concurrent
 * streams, threads) race; serialise them.
 * No counterpart in the reference: for callers that cannot allocate or
 * manage a workspace (code under graph capture, tight serving loops,
 * harnesses that forbid hipMalloc). */
int bmx_qmatmul_affine_noalloc(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales,
                               const bmx_bf16 *biases, bmx_bf16 *y, int64_t M, int64_t N, int64_t K,
                               int transpose, int group_size, int bits, void *stream);

/* Routed (MoE expert) quantized matmul: w [n_experts, N, K/8] u32, scales /
 * biases [n_experts, N, K/64] bf16; for route r < n_routes,
 *   out[r] [M, N] = x[r / x_bcast] [M, K] . W[rhs_indices[r]]^T
 * with quantized_matmul's numerics (fp32 accumulate, bf16 out).  x holds
 * n_routes / x_bcast row blocks of [M, K] (x_bcast = top_k when every slot
 * of a token shares its x, 1 for one block per route).  rhs_indices is a
 * device array of n_routes uint32; ids >= n_experts are clamped to
 * n_experts - 1.  M <= 8, K % 64 == 0, n_routes <= 65535; x and w 16-byte
 * aligned.
 * Replaces: mlx_ext::gather_qmm(x, w, scales, biases, None, Some(indices),
 *   transpose=true, gs, bits, sorted=false) (crates/base-mlx-core/src/
 *   mlx_ext.rs:66-117) as called by QSwitchLinear::forward
 *   (crates/base-mlx-core/src/model/granite.rs:74-88). */
int bmx_gather_qmm(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales, const bmx_bf16 *biases,
                   const uint32_t *rhs_indices, bmx_bf16 *out, int n_routes, int x_bcast, int n_experts, int M,
                   int N, int K, int group_size, int bits, void *stream);
/* bmx_gather_qmm with mlx_gather_qmm's whole argument list: for route
 * r < n_routes,
 *   out[r] [M, N] = x[lhs(r)] [M, K] . W[rhs(r)]^T
 * x holds n_x_blocks row blocks of [M, K].  lhs(r) = lhs_indices[r] (device
 * uint32; ids >= n_x_blocks are clamped to n_x_blocks - 1), or, with
 * lhs_indices NULL, r / (n_routes / n_x_blocks) (n_x_blocks must divide
 * n_routes).  rhs(r) = rhs_indices[r] (device uint32; ids >= n_experts are
 * clamped to n_experts - 1), or, with rhs_indices NULL, r (n_routes must
 * equal n_experts).  transpose must be 1 (BMX_E_UNSUPPORTED otherwise);
 * sorted_indices only says the routes come grouped by expert and does not
 * change the results.  Other limits as bmx_gather_qmm.
 * Replaces: mlx_ext::gather_qmm(x, w, scales, biases, lhs_indices,
 *   rhs_indices, transpose, group_size, bits, sorted_indices)
 *   (crates/base-mlx-core/src/mlx_ext.rs:66-117). */
int bmx_gather_qmm_indexed(const bmx_bf16 *x, const uint32_t *w, const bmx_bf16 *scales, const bmx_bf16 *biases,
                           const uint32_t *lhs_indices, const uint32_t *rhs_indices, bmx_bf16 *out, int n_routes,
                           int n_x_blocks, int n_experts, int M, int N, int K, int transpose, int group_size,
                           int bits, int sorted_indices, void *stream);

/* out[N,K] = scales * q + biases (fp32, rounded to bf16).
 * Replaces: mlx_rs::ops::dequantize(w, s, b, group_size, bits)
 *   (crates/base-mlx-core/src/model/qwen3.rs:75). */
int bmx_dequantize_affine(const uint32_t *w, const bmx_bf16 *scales, const bmx_bf16 *biases,
                          bmx_bf16 *out, int64_t N, int64_t K, int group_size, int bits,
                          void *stream);

/* out[m,:] = dequantize(row ids[m] of (w, scales, biases)), m < M.
 * ids are int32 token ids in [0, rows); an id outside that range yields a
 * zero row.
 * Replaces: QEmbedding::lookup = index(tokens) + dequantize
 *   (crates/base-mlx-core/src/model/qwen3.rs:67-76). */
int bmx_dequant_gather(const int32_t *ids, int64_t M, int64_t rows, const uint32_t *w,
                       const bmx_bf16 *scales, const bmx_bf16 *biases, bmx_bf16 *out, int64_t K,
                       int group_size, int bits, void *stream);

/* ------------------------------------------------------------------ */
/* Seeded random initialisation (the benchmark workloads use random-init */
/* weights; these kernels are bit-identical to the CPU generator).      */
/* No counterpart in the reference, which loads weights from            */
/* safetensors (crates/base-mlx-core/src/model/qwen3.rs:194-295).       */
/* ------------------------------------------------------------------ */

/* Element (n,k) = t * c with t the centred sum of the four 16-bit fields
 * of rand64(seed, n*K + k) (approx normal), quantized to MLX affine 4-bit
 * gs64 with the documented formula evaluated exactly on the integers t:
 * q = rne(15 (t - tmin) / (tmax - tmin)), s = (tmax - tmin) c / 15,
 * b = tmin c (the group minimum). */
int bmx_init_qlinear(uint64_t seed, int64_t N, int64_t K, float c, uint32_t *w,
                     bmx_bf16 *scales, bmx_bf16 *biases, void *stream);
/* out[i] = bf16(approx-normal(seed, i) * c) */
int bmx_fill_normal_bf16(uint64_t seed, int64_t n, float c, bmx_bf16 *out, void *stream);

/* ------------------------------------------------------------------ */
/* Ops of a Qwen3 attention / MLP block                                 */
/* ------------------------------------------------------------------ */

/* y[r,:] = w * bf16(x[r,:] * rsqrt(mean(x[r,:]^2) + eps)), fp32 inside;
 * dim % 8 == 0, 16-byte aligned pointers.
 * Replaces: mlx_rs::fast::rms_norm via RmsNorm::forward
 *   (crates/base-mlx-core/src/model/qwen3.rs:44-55). */
int bmx_rms_norm(const bmx_bf16 *x, const bmx_bf16 *w, bmx_bf16 *y, int64_t rows, int64_t dim, float eps,
                 void *stream);

/* Rotate-half RoPE over [H, T, D]: for i < D/2, angle = (offset + t) *
 * theta^(-i/(D/2)); y may alias x.
 * Replaces: mlx_rs::fast::rope(x, D, traditional=false, theta, 1.0, offset)
 *   (crates/base-mlx-core/src/model/qwen3.rs:410-413). */
int bmx_rope(const bmx_bf16 *x, bmx_bf16 *y, int64_t H, int64_t T, int64_t D, float theta, int64_t offset,
             void *stream);

/* In place: src[start[d]:stop[d]:strides[d] for each axis d] = update
 * (numpy semantics, positive strides, ndim <= 8).  shape/start/stop/strides
 * are HOST arrays; src and update are device bf16.
 * Replaces: mlx_ext::slice_update(src, update, start, stop, strides)
 *   (crates/base-mlx-core/src/mlx_ext.rs:36-64) -- always in place. */
int bmx_slice_update(bmx_bf16 *src, int ndim, const int64_t *shape, const bmx_bf16 *update,
                     const int64_t *start, const int64_t *stop, const int64_t *strides, void *stream);

/* Fused QK-norm + RoPE + KV write for M new tokens at cache position
 * `offset` (head_dim 128):  q [M, n_heads*128], k, v [M, n_kv_heads*128]
 * (projection outputs) -> q_out [n_heads, M, 128] (normed, rotated) and
 * k_cache/v_cache [n_kv_heads, capacity, 128] rows offset..offset+M-1.
 * offset + M > capacity returns BMX_E_KV_CAPACITY and writes nothing.
 * Replaces: the per-layer sequence of Qwen3::forward_internal
 *   q_norm/k_norm -> transpose -> fast::rope -> mlx_ext::slice_update
 *   (crates/base-mlx-core/src/model/qwen3.rs:392-489). */
int bmx_qk_norm_rope_kv(const bmx_bf16 *q, const bmx_bf16 *k, const bmx_bf16 *v, const bmx_bf16 *q_norm,
                        const bmx_bf16 *k_norm, bmx_bf16 *q_out, bmx_bf16 *k_cache, bmx_bf16 *v_cache, int M,
                        int n_heads, int n_kv_heads, int head_dim, int capacity, int offset, float eps,
                        float theta, void *stream);

/* GQA attention of M queries q [n_heads, M, 128] over keys/values
 * k_cache, v_cache [n_kv_heads, capacity, 128] rows 0..offset+M-1:
 * out [M, n_heads*128] = softmax(scale q k^T + mask) v, query head h using
 * kv head h / (n_heads / n_kv_heads); for M > 1 query t sees keys
 * j <= offset + t.  `workspace` (may be NULL: no key split) holds arrival
 * counters and split partials; bmx_attention_workspace_bytes(n_heads, M) is
 * enough, 16-byte aligned.  It must be zero-filled before its first use; every call leaves
 * the counters zero again, so it is reused as is.  Calls that share one
 * workspace must not run concurrently.
 * Replaces: mlx_rs::fast::scaled_dot_product_attention with the
 *   causal_mask_offset mask (crates/base-mlx-core/src/model/qwen3.rs:491-518,
 *   629-653). */
int bmx_attention_gqa(const bmx_bf16 *q, const bmx_bf16 *k_cache, const bmx_bf16 *v_cache, bmx_bf16 *out,
                      int n_heads, int n_kv_heads, int M, int head_dim, int capacity, int offset, float scale,
                      void *workspace, size_t workspace_bytes, void *stream);
size_t bmx_attention_workspace_bytes(int n_heads, int M);

/* bmx_qk_norm_rope_kv followed by bmx_attention_gqa, as one kernel: q, k, v
 * are the raw projection rows [M, n_heads*128] / [M, n_kv_heads*128]; the
 * new keys and values go to k_cache / v_cache rows offset..offset+M-1 as
 * bmx_qk_norm_rope_kv writes them, and out is bit-identical to the two-call
 * sequence (the normed q itself is not stored).  Needs M <= 16,
 * M * (n_heads / n_kv_heads) <= 64 and a zero-filled workspace as for
 * bmx_attention_gqa (else BMX_E_UNSUPPORTED, nothing written).
 * Replaces: the same per-layer sequence of Qwen3::forward_internal
 *   (crates/base-mlx-core/src/model/qwen3.rs:392-518) on decode and
 *   speculative-verify steps. */
int bmx_qk_norm_rope_kv_attention(const bmx_bf16 *q, const bmx_bf16 *k, const bmx_bf16 *v, const bmx_bf16 *q_norm,
                                  const bmx_bf16 *k_norm, bmx_bf16 *k_cache, bmx_bf16 *v_cache, bmx_bf16 *out, int M,
                                  int n_heads, int n_kv_heads, int head_dim, int capacity, int offset, float eps,
                                  float theta, float scale, void *workspace, size_t workspace_bytes, void *stream);

/* out[r] = index of the max of x[r, 0:n] (first index on ties), uint32.
 * Replaces: argmax / argmax_axis in pick_next and the speculative loop
 *   (crates/base-mlx-core/src/engine.rs:195-202;
 *   crates/base-mlx-core/src/speculative.rs:168-173, 289-293). */
int bmx_argmax_rows(const bmx_bf16 *x, int64_t rows, int64_t n, uint32_t *out, void *stream);

/* y = bf16(bf16(g * bf16(sigmoid(g))) * up), elementwise.
 * Replaces: nn::silu(gate) * up in mlp_block
 *   (crates/base-mlx-core/src/model/kernels.rs:73-74). */
int bmx_silu_mul(const bmx_bf16 *gate, const bmx_bf16 *up, bmx_bf16 *y, int64_t n, void *stream);
/* y = bf16(a + b); y may alias a or b.
 * Replaces: the residual adds `&x + &attn`, `&x + &mlp_out[0]`
 *   (crates/base-mlx-core/src/model/qwen3.rs:521, 541). */
int bmx_add(const bmx_bf16 *a, const bmx_bf16 *b, bmx_bf16 *y, int64_t n, void *stream);

/* ------------------------------------------------------------------ */
/* Qwen3 model, KV cache, generation                                   */
/* ------------------------------------------------------------------ */

/* Shape parameters (ModelConfig, crates/base-mlx-core/src/model/config.rs:11-201). */
typedef struct {
  int hidden, inter, layers, n_heads, n_kv_heads, head_dim, vocab;
  int tied;              /* tie_word_embeddings */
  int group_size, bits;  /* quantization: 64, 4 */
  float eps, rope_theta;
} bmx_qwen3_config;

typedef struct bmx_qwen3 bmx_qwen3;
typedef struct bmx_kv_cache bmx_kv_cache;

/* A Qwen3 with seeded random-init weights (projections approx N(0, sigma)
 * quantized as bmx_init_qlinear, norms 1) and workspace for forwards of up
 * to max_tokens tokens.
 * Replaces: Qwen3::load (crates/base-mlx-core/src/model/qwen3.rs:194-295) for
 *   the benchmark workloads, which use random-init weights. */
int bmx_qwen3_create_random(const bmx_qwen3_config *cfg, uint64_t seed, double sigma, int max_tokens,
                            bmx_qwen3 **out);
void bmx_qwen3_destroy(bmx_qwen3 *model);

/* HuggingFace config.json -> shape parameters: `quantization` and
 * `quantization_config` merged (the first wins), num_key_value_heads
 * defaulting to num_attention_heads, head_dim to hidden / heads,
 * rms_norm_eps to 1e-6, rope_theta to 10000, tie_word_embeddings to false;
 * a model_type other than "qwen3" is BMX_E_UNSUPPORTED.  Host only.
 * Replaces: ModelConfig::from_path (crates/base-mlx-core/src/model/config.rs:
 *   149-167, defaults config.rs:109-135, 184-191). */
int bmx_qwen3_config_from_json(const char *path, bmx_qwen3_config *out);

/* A Qwen3 from an MLX checkpoint directory: config.json plus every
 * *.safetensors shard (sorted; a later shard overrides a name), tensors taken
 * by their MLX names (model.embed_tokens.{weight,scales,biases},
 * model.layers.{i}.self_attn.{q,k,v,o}_proj.*, .mlp.{gate,up,down}_proj.*,
 * .self_attn.{q,k}_norm.weight, .input_layernorm.weight,
 * .post_attention_layernorm.weight, model.norm.weight, lm_head.* when
 * untied).  Packed weights U32 (or I32); scales, biases, norms BF16, or
 * F16 / F32 rounded to bf16.  A missing tensor, a shape that disagrees with
 * the config, or tensors left over are errors (BMX_E_SHAPE, the message
 * names them), all found before any GPU allocation.
 * Replaces: Qwen3::load with read_all_shards (crates/base-mlx-core/src/model/
 *   qwen3.rs:194-295, 580-627) and the bits check of infer_bits
 *   (crates/base-mlx-core/src/model/gemma.rs:760-779). */
int bmx_qwen3_load(const char *dir, int max_tokens, bmx_qwen3 **out);
/* Device pointers of a projection: layer >= 0 with slot 0..6 = q,k,v,o,
 * gate,up,down; layer -1 = embed_tokens; layer -2 = lm head (tied: embed).
 * Mirrors the tensor map of Qwen3::load (qwen3.rs:205-273).  A layer
 * projection may be written through them: the next forward of more than 8
 * tokens first rewrites the group-major copies its GEMMs read. */
int bmx_qwen3_qlinear(bmx_qwen3 *model, int layer, int slot, uint32_t **w, bmx_bf16 **scales,
                      bmx_bf16 **biases, int *N, int *K);

/* KV cache [layers, 2, n_kv_heads, capacity, 128] bf16, zero-filled.
 * Replaces: KvCache (crates/base-mlx-core/src/model/qwen3.rs:109-162) with the
 *   capacity a parameter instead of KV_PREALLOC (qwen3.rs:125). */
int bmx_kv_create(const bmx_qwen3 *model, int capacity, bmx_kv_cache **out);
void bmx_kv_destroy(bmx_kv_cache *cache);
int bmx_kv_seq_len(const bmx_kv_cache *cache);
int bmx_kv_capacity(const bmx_kv_cache *cache);
/* KvCache::reset (qwen3.rs:131-135) */
void bmx_kv_reset(bmx_kv_cache *cache);
/* KvCache::truncate (qwen3.rs:150-161): no-op if target >= seq_len; keeps
 * the preallocated buffer (only seq_len moves). */
void bmx_kv_truncate(bmx_kv_cache *cache, int target);
bmx_bf16 *bmx_kv_data(bmx_kv_cache *cache);
/* Positions [0, seq_len) of every K/V row <- approx N(0,1) (counter
 * (row * capacity + t) * 128 + d); sets seq_len.  Synchronises `stream`.
 * No counterpart in the reference: a stand-in for a long prefill when
 * only later decode steps are measured. */
int bmx_kv_fill_synthetic(bmx_kv_cache *cache, uint64_t seed, int seq_len, void *stream);

/* Forward of M tokens (HOST array) at position seq_len; logits (device)
 * [M, vocab] if all_logits else [1, vocab] (last row); seq_len += M.
 * Errors (no state change): BMX_E_KV_CAPACITY if seq_len + M > capacity,
 * BMX_E_SHAPE on a cache/model mismatch, BMX_E_ARG on a token >= vocab.
 * Replaces: Qwen3::forward / forward_multi
 *   (crates/base-mlx-core/src/model/qwen3.rs:302-312). */
int bmx_qwen3_forward(bmx_qwen3 *model, bmx_kv_cache *cache, const uint32_t *tokens, int M, int all_logits,
                      bmx_bf16 *logits, void *stream);
/* One decode step for `token` through the captured decode graph; writes
 * the greedy next token to *next_token (host) and, if logits != NULL, the
 * logits (device [vocab]).  Synchronises the stream.
 * Replaces: Qwen3::forward(&[next]) + pick_next (engine.rs:114-124, 195-202). */
int bmx_qwen3_decode_step(bmx_qwen3 *model, bmx_kv_cache *cache, uint32_t token, uint32_t *next_token,
                          bmx_bf16 *logits, void *stream);
/* Greedy generation: prefill `prompt` (host, P tokens), then decode until
 * an eos token (not emitted) or max_new tokens; out (host) receives the
 * tokens, *n_out their count.
 * Replaces: LoadedModel::generate_text with temperature 0
 *   (crates/base-mlx-core/src/engine.rs:100-144, 146-153, 217-223). */
int bmx_generate_greedy(bmx_qwen3 *model, bmx_kv_cache *cache, const uint32_t *prompt, int P, int max_new,
                        const uint32_t *eos, int n_eos, uint32_t *out, int *n_out, void *stream);
/* The decode loop of bmx_generate_greedy alone, continuing a cache whose
 * prefill picked `token` (the first generated token, at position seq_len):
 * emits `token` unless it is an eos token, then decodes one token per step
 * from the last one emitted, until an eos token (not emitted) or max_new
 * tokens in all; out (host, max_new entries) receives them, *n_out their
 * count, and seq_len advances by the steps taken.  Steps are queued on the
 * stream ahead of the token being checked; on return the stream is
 * synchronised and the cache holds exactly the steps the loop took.
 * BMX_E_KV_CAPACITY (with *n_out tokens written) at the step that would not
 * fit, as bmx_qwen3_decode_step would return it.
 * Replaces: the loop of LoadedModel::generate / generate_text with
 *   temperature 0 (crates/base-mlx-core/src/engine.rs:103-115). */
int bmx_decode_greedy(bmx_qwen3 *model, bmx_kv_cache *cache, uint32_t token, int max_new, const uint32_t *eos,
                      int n_eos, uint32_t *out, int *n_out, void *stream);
/* Greedy speculative decoding with verify width spec_k (leader + spec_k-1
 * drafts; the reference fixes SPEC_K = 4).  out needs max_new entries;
 * stats (optional, 3 entries): iterations, proposed, accepted.
 * Replaces: speculative::generate (crates/base-mlx-core/src/speculative.rs:57-286). */
int bmx_speculative_generate(bmx_qwen3 *target, bmx_kv_cache *target_cache, bmx_qwen3 *draft,
                             bmx_kv_cache *draft_cache, const uint32_t *prompt, int P, int max_new, int spec_k,
                             const uint32_t *eos, int n_eos, uint32_t *out, int *n_out, int64_t *stats,
                             void *stream);

#ifdef __cplusplus
}
#endif
#endif /* BMX_H */
