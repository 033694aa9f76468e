/* wave_hip_attn.h -- C ABI of the MI355X (gfx950) causal attention tier.
 *
 * This is the drop-in boundary for wave-engine's ComputeBackend attention
 * methods (reference: src/common/compute.rs:8-174).  Everything is plain C:
 * raw pointers, sizes and a `void*` HIP stream; no Rust, torch or HIP types
 * appear in a signature, so a Rust `extern "C"` block (or ctypes) binds it
 * directly.
 *
 * Conventions
 *   - Every function returns 0 (WHA_OK) or a negative WHA_ERR_* code; the
 *     message for the calling thread's last failure is wha_last_error().
 *     The reference's methods are infallible and panic on failure
 *     (e.g. src/wgpu_tier/pipelines.rs:138); a Rust shim turns a non-zero
 *     return into panic!(wha_last_error()).
 *   - Device entry points take device pointers, enqueue on `stream`
 *     (NULL = the null stream) and return without synchronising.
 *   - Host entry points take host pointers in the reference's per-sequence
 *     layout and return after the results are in host memory.
 *   - All tensors are fp32.  Arithmetic is fp32 throughout (MFMA
 *     v_mfma_f32_16x16x4_f32 for the contractions).
 *   - Entry points are re-entrant and may be called from several host
 *     threads at once (the reference calls the backend from one thread per
 *     batch element, src/cpu/train_loop.rs:320-365).
 */
#ifndef WAVE_HIP_ATTN_H
#define WAVE_HIP_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WHA_OK 0
#define WHA_ERR_INVALID (-1)     /* bad shape, stride, pointer or scale      */
#define WHA_ERR_UNSUPPORTED (-2) /* head_dim > 128 or similar limits         */
#define WHA_ERR_HIP (-3)         /* a HIP runtime call failed                */
#define WHA_ERR_WORKSPACE (-4)   /* caller workspace too small               */
#define WHA_ERR_NOMEM (-5)       /* device or host allocation failed         */

/* Strided view of B*H independent [T][D] matrices: element (b,h,t,d) of a
 * tensor with base pointer p is p[b*stride_b + h*stride_h + t*stride_t + d]
 * (unit stride on d).  One layout describes q, k, v, o, do, dq, dk and dv.
 *   device layout [B,H,T,D] contiguous: stride_b=H*T*D, stride_h=T*D, stride_t=D
 *   reference per-sequence layout [T][H*D] (src/common/compute.rs:370-374,
 *   :384-386) batched as [B][T][H*D]: stride_b=T*H*D, stride_h=D, stride_t=H*D
 * Rows of distinct (b,h,t) must not overlap (the layout also describes the
 * outputs): taken in increasing stride order, each dimension of extent > 1
 * must step at least over the span of the smaller ones, else WHA_ERR_INVALID
 * (zero strides, i.e. K or V shared across heads, are rejected).
 * lse is always [B][H][T] contiguous; workspaces are opaque scratch whose
 * size the matching *_workspace_size function reports. */
typedef struct wha_layout {
  int32_t B, H, T, D;
  int64_t stride_b, stride_h, stride_t;
} wha_layout;

/* Thread-local message of this thread's last failed call ("" if none). */
const char* wha_last_error(void);

/* Library version string. */
const char* wha_version(void);

/* ---------------------------------------------------------------- device API */

/* Fused causal forward: o = softmax(q k^T * scale, causal) v, per (b,h), and
 * lse[b][h][t] = log(sum_{j<=t} exp(q_t.k_j*scale)) (natural log).  The T x T
 * score matrix is never materialised.  lse may be NULL when no backward will
 * follow.  Replaces the core of attention_cpu (src/common/compute.rs:377-409)
 * and the host loops of GpuBackend::attention (src/wgpu_tier/dispatch.rs:106-136).
 * scale is normally 1/sqrt(D) (src/common/compute.rs:362). */
int wha_attn_fwd(const float* q, const float* k, const float* v, float* o,
                 float* lse, const wha_layout* layout, float scale,
                 void* stream);

/* Bytes of device workspace wha_attn_bwd needs for this layout: per-row
 * statistics (Delta_t = dO_t . O_t, and for head dim 64 the scaled LSE beside
 * it, in 32-row blocks) plus the causal half of dS in 64-key column blocks,
 * which the key-stationary pass writes and the dQ pass reads. */
size_t wha_attn_bwd_workspace_size(const wha_layout* layout);

/* Fused causal backward from the forward's o and lse: recomputes P on chip and
 * writes dq, dk, dv (overwritten, not accumulated).  workspace may be NULL, in
 * which case the library uses a cached device buffer of its own, one per
 * (host thread, device, stream), grown on demand; calls that share a thread
 * and a stream are ordered by the stream, so they never race on it.  Valid when the att the
 * caller would have passed is causal softmax(q k^T * scale), which is the only
 * way the reference produces it.  Replaces attn_backward_scores +
 * attn_backward_dkv (shaders/attn_backward_scores.wgsl:27-111,
 * shaders/attn_backward_dkv.wgsl:22-63) as driven by
 * src/wgpu_tier/dispatch_backward.rs:328-436, and the math of
 * attention_backward_single (src/cpu/backward.rs:313-363). */
int wha_attn_bwd(const float* q, const float* k, const float* v,
                 const float* o, const float* d_o, const float* lse, float* dq,
                 float* dk, float* dv, void* workspace, size_t workspace_bytes,
                 const wha_layout* layout, float scale, void* stream);

/* Training pair that keeps the forward's scores for the backward, as the
 * reference's forward keeps its attention weights and hands them to
 * attention_backward (src/common/compute.rs:391-399 -> :286-314,
 * src/cpu/backward.rs:330).  wha_attn_fwd_keep is wha_attn_fwd that also
 * writes the raw scores q_t.k_j*scale*log2(e) of the causal half into scores;
 * wha_attn_bwd_kept is wha_attn_bwd that reads them instead of recomputing
 * q k^T (same workspace as wha_attn_bwd).  scores: wha_attn_scores_size bytes
 * of device memory, 16-byte aligned, opaque (its layout is internal), valid
 * until the next wha_attn_fwd_keep into it.  When wha_attn_scores_size is 0
 * (head dims outside 36..128 or not a multiple of 4, strides not multiples of
 * 4 floats, a problem small enough for the split-sweep kernels -- fewer than
 * 256 64-row tiles over all heads, T <= 1024 -- or a score buffer above
 * 8 GiB) scores may be NULL and the pair
 * behaves exactly as wha_attn_fwd / wha_attn_bwd.  The pair also runs as
 * wha_attn_fwd / wha_attn_bwd when a tensor is not 16-byte aligned (the
 * forward then leaves scores untouched).  The library records, per score
 * buffer, whether the last wha_attn_fwd_keep into it wrote scores and for
 * which B, H, T, D; wha_attn_bwd_kept reads scores only when that record says
 * so (and its own tensors are aligned), and otherwise recomputes them, so a
 * backward never reads scores the forward did not write.  scores itself, when
 * used, must be non-NULL and 16-byte aligned (WHA_ERR_INVALID if not). */
size_t wha_attn_scores_size(const wha_layout* layout);
int wha_attn_fwd_keep(const float* q, const float* k, const float* v, float* o,
                      float* lse, float* scores, const wha_layout* layout,
                      float scale, void* stream);
int wha_attn_bwd_kept(const float* q, const float* k, const float* v,
                      const float* o, const float* d_o, const float* lse,
                      const float* scores, float* dq, float* dk, float* dv,
                      void* workspace, size_t workspace_bytes,
                      const wha_layout* layout, float scale, void* stream);

/* Bytes of device workspace wha_attn_bwd_from_probs needs. */
size_t wha_attn_bwd_from_probs_workspace_size(const wha_layout* layout);

/* Backward with the reference's exact contract: att [B][H][T][T] (post-softmax
 * rows; entries j > t never reach the result and may hold anything, NaN
 * included) is used as given and never
 * recomputed, exactly as ComputeBackend::attention_backward
 * (src/common/compute.rs:163-173, :286-314) and attention_backward_single
 * (src/cpu/backward.rs:313-363) use it.  d_pre_proj is the gradient flowing
 * into the pre-c_proj attention output.  Workspace: Delta plus the dS tiles
 * (as wha_attn_bwd); the causal half of att is streamed twice (the Delta pass
 * and the dK/dV pass). */
int wha_attn_bwd_from_probs(const float* d_pre_proj, const float* q,
                            const float* k, const float* v, const float* att,
                            float* dq, float* dk, float* dv, void* workspace,
                            size_t workspace_bytes, const wha_layout* layout,
                            float scale, void* stream);

/* Bytes of device workspace wha_decode_fwd needs (split-K partials). */
size_t wha_decode_workspace_size(const wha_layout* cache_layout);

/* Single-token decode: for each (b,h), one query q[b][h][:] (q and o are
 * [B][H][D] contiguous) attends to every one of the T cached keys of
 * k_cache/v_cache (described by cache_layout, T = cache length).  Equals the
 * last row of a causal pass with T = cache length.  lse ([B][H]) may be NULL.
 * The reference has no dot-product decode; the nearest analogue is
 * kv_cache::forward_one (src/common/kv_cache.rs:241-356). */
int wha_decode_fwd(const float* q, const float* k_cache, const float* v_cache,
                   float* o, float* lse, void* workspace, size_t workspace_bytes,
                   const wha_layout* cache_layout, float scale, void* stream);

/* wha_decode_fwd that allocates nothing, for callers that cannot call
 * hipMalloc (code under HIP graph capture, tight serving loops, harnesses that
 * forbid allocation).  No counterpart in the reference: it exists for those
 * callers only.  The split-K partials live in a static device array of
 * 16 MiB that every GPU the library runs on holds until the process ends;
 * layouts whose partials need more (wha_decode_workspace_size above 16 MiB,
 * e.g. B*H = 768 at D = 64 beyond about 82 000 cached keys) return
 * WHA_ERR_WORKSPACE before any pointer is looked at.  All calls on one GPU
 * share that array: calls that overlap on one GPU (several streams or host
 * threads at once) race and must be serialised by the caller.  Otherwise the
 * same contract and results as wha_decode_fwd. */
int wha_decode_fwd_noalloc(const float* q, const float* k_cache,
                           const float* v_cache, float* o, float* lse,
                           const wha_layout* cache_layout, float scale,
                           void* stream);

/* Rows of the attention probabilities on demand, for consumers of materialised
 * P: the head monitor reads the last row of every head
 * (src/monitors/attn_monitor.rs:26-80) and the softmax_rows value contract
 * checks rows in [0, 1] that sum to 1 (src/monitors/junctions/value_range.rs:117-121).
 * Recomputed from q, k and the forward's lse:
 *   out[b][h][r][j] = exp(q_t . k_j * scale - lse[b][h][t]) for j <= t = rows[r], 0 for j > t.
 * rows is a host array of n_rows (1..256) query indices in [0, T); out is
 * [B][H][n_rows][T] contiguous. */
int wha_attn_probs_rows(const float* q, const float* k, const float* lse,
                        const int32_t* rows, int32_t n_rows, float* out,
                        const wha_layout* layout, float scale, void* stream);

/* ---------------------------------------------------------------- projections
 * The c_attn / c_proj linears around the core (fp32 MFMA GEMM).  A batch of M
 * rows is one call; rows of x / y / dy / dx have the given strides (floats),
 * w is [N][K] row-major ([out_dim][in_dim], LinearWeights src/common/model.rs:175-180). */

/* y[m][n] = b[n] + sum_k w[n][k] x[m][k]  (b may be NULL: no bias).
 * ComputeBackend::linear_batch / linear_no_bias_batch (src/common/compute.rs:56-61,
 * :441-468); one row is linear (src/common/model.rs:144-151). */
int wha_linear_fwd(const float* x, int64_t ldx, const float* w, const float* b,
                   float* y, int64_t ldy, int64_t M, int32_t N, int32_t K,
                   void* stream);

/* dx[m][k] = sum_n dy[m][n] w[n][k].  ComputeBackend::linear_backward_dx_batch
 * (src/common/compute.rs:150, linear_backward_dx_only src/common/math/backward.rs:36-46). */
int wha_linear_bwd_dx(const float* dy, int64_t lddy, const float* w, float* dx,
                      int64_t lddx, int64_t M, int32_t N, int32_t K,
                      void* stream);

/* Bytes of device workspace wha_linear_bwd_dw needs. */
size_t wha_linear_bwd_dw_workspace_size(int64_t M, int32_t N, int32_t K);

/* dw[n][k] = sum_m dy[m][n] x[m][k] and, when db != NULL, db[n] = sum_m dy[m][n]
 * (overwritten, summed in a fixed order).  ComputeBackend::outer_product_accum
 * (src/common/compute.rs:153-161, :263-282) with compute_bias = (db != NULL).
 * workspace may be NULL (library-cached, as for wha_attn_bwd). */
int wha_linear_bwd_dw(const float* dy, int64_t lddy, const float* x, int64_t ldx,
                      float* dw, float* db, int64_t M, int32_t N, int32_t K,
                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- host API
 * One sequence in the reference's layout: q, k, v, o, d_pre_proj, dq, dk, dv
 * are [T][E] row-major host arrays (E = n_head * head_dim), att is
 * [n_head][T][T].  scale = 1/sqrt(E/n_head) as the reference computes it.
 * Synchronous; device buffers are staged through a per-thread cache. */

/* Core of attention_cpu (src/common/compute.rs:377-409): o = causal softmax
 * attention of q,k,v (the c_attn/c_proj linears around it are not included). */
int wha_host_attention_core_fwd(const float* q, const float* k, const float* v,
                                int32_t T, int32_t E, int32_t n_head, float* o);

/* ComputeBackend::attention (src/common/compute.rs:42-43) = attention_cpu
 * (:357-414) end to end: qkv = c_attn(x) (:368-375), causal attention core,
 * out = c_proj(o) (:411-413).  x, out: [T][E]; c_attn_w [3E][E], c_attn_b [3E],
 * c_proj_w [E][E], c_proj_b [E] (AttentionWeights, src/common/model.rs:189-195). */
int wha_host_attention(const float* x, const float* c_attn_w,
                       const float* c_attn_b, const float* c_proj_w,
                       const float* c_proj_b, int32_t T, int32_t E,
                       int32_t n_head, float* out);

/* ComputeBackend::attention_backward (src/common/compute.rs:163-173) with
 * CpuBackend's semantics (:286-314): att used as given. */
int wha_host_attention_backward(const float* d_pre_proj, const float* q,
                                const float* k, const float* v,
                                const float* att, int32_t T, int32_t E,
                                int32_t n_head, float* dq, float* dk,
                                float* dv);

/* ---------------------------------------------------------------- wave attention
 * The harmonic coherence attention the reference trains with
 * (src/common/attn.rs:72-430; callers src/cpu/forward.rs:113 and
 * src/cpu/model_backward.rs:380-395).  Device pointers, batched over B
 * sequences of T positions, input x [B][T][n_embd] contiguous (the normed
 * hidden state the reference passes in). */

/* Shape.  content_dim C = rows of each head's content projection (0 = none,
 * the reference's backward-compatible mode; at most 30); head_dim =
 * n_embd / n_head must be at most 128. */
typedef struct wha_wave_shape {
  int32_t B, T, n_embd, n_head, content_dim;
} wha_wave_shape;

/* Weights (WaveAttnWeights, attn.rs:17-46), device pointers, fp32:
 *   harmonic_raw [n_head]
 *   proj_w [n_head][2 + C][n_embd]: row 0 / 1 = phase_proj_w[0] / [1] (r, s),
 *          rows 2 .. 1+C = content_proj_w   (one GEMM computes all of them)
 *   proj_b [n_head][2 + C]: phase_proj_b then content_proj_b
 *   v_w [n_head][head_dim][head_dim], v_b [n_head][head_dim]
 *   out_w [n_embd][n_embd], out_b [n_embd] */
typedef struct wha_wave_weights {
  const float* harmonic_raw;
  const float* proj_w;
  const float* proj_b;
  const float* v_w;
  const float* v_b;
  const float* out_w;
  const float* out_b;
} wha_wave_weights;

/* Forward intermediates kept for the backward (the role of WaveAttnCache,
 * attn.rs:48-70), caller-allocated device buffers:
 *   proj   [B][T][n_head][2 + C]  r, s and the content vector
 *   values [B][T][n_embd]         per-head value projections (head h at columns h*head_dim)
 *   feat   [B][n_head][T][32]     cos(n phi), sin(n phi), content, zeros (16-byte aligned)
 *   phase  [B][n_head][T]         phi = atan2(s, r)
 *   bucket [B][n_head][T]         phase_to_bucket(phi) (kv_cache.rs:66-70)
 *   merged [B][T][n_embd]         head outputs before out_proj (out_merged)
 *   lse    [B][n_head][T]         natural-log row log-sum-exp of the scores */
typedef struct wha_wave_cache {
  float* proj;
  float* values;
  float* feat;
  float* phase;
  int32_t* bucket;
  float* merged;
  float* lse;
} wha_wave_cache;

/* Workspace bytes of wha_wave_fwd: the bucket-sparse family's sorted operand
 * copies, whenever the shape can take that family whatever the mode set by
 * wha_wave_set_bucket_sparse (0 for an invalid shape, or one that only runs
 * the all-pairs family). */
size_t wha_wave_fwd_workspace_size(const wha_wave_shape* shape);

/* wave_attention_forward (attn.rs:90-305): out [B][T][n_embd] and the cache.
 * The reference's att_weights_all is not materialised; wha_wave_probs_rows
 * recomputes any rows of it from the cache.  workspace: at least
 * wha_wave_fwd_workspace_size bytes, 16-byte aligned, scratch for this call
 * only.  With workspace NULL the bucket-sparse family (the default from
 * T = 1024) takes a library-cached buffer per (host thread, device, stream),
 * as wha_attn_bwd does: growing it synchronises the stream and calls
 * hipFree / hipMalloc, so callers that cannot allocate (HIP graph capture,
 * allocation-free loops) must pass a workspace.  The all-pairs family needs
 * none and never allocates. */
int wha_wave_fwd(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape, float* out,
                 const wha_wave_cache* cache, void* workspace, size_t workspace_bytes, void* stream);

/* Gradients.  d_x [B][T][n_embd] (d_normed) is required; the weight
 * gradients (same layouts as wha_wave_weights, summed over the B sequences)
 * are either all non-NULL (wave_attention_backward_full, attn.rs:346-430) or
 * all NULL (wave_attention_backward_pathway, attn.rs:432-511: d_x only). */
typedef struct wha_wave_grads {
  float* d_x;
  float* d_harmonic_raw;
  float* d_proj_w;
  float* d_proj_b;
  float* d_v_w;
  float* d_v_b;
  float* d_out_w;
  float* d_out_b;
} wha_wave_grads;

/* Workspace bytes of wha_wave_bwd (0 for an invalid shape). */
size_t wha_wave_bwd_workspace_size(const wha_wave_shape* shape);

/* Backward from d_out = d_attn_out [B][T][n_embd] (the gradient of out), the
 * forward's x and cache.  Deterministic (no atomics). */
int wha_wave_bwd(const float* x, const float* d_out, const wha_wave_weights* w, const wha_wave_shape* shape,
                 const wha_wave_cache* cache, const wha_wave_grads* grads, void* workspace,
                 size_t workspace_bytes, void* stream);

/* Rows of att_weights_all (attn.rs:240, :259-269) on demand, from the cache:
 * out[b][h][r][j] for query t = rows[r] is the post-softmax weight of key j
 * (0 where the bucket mask excludes j <= t, -inf for j > t as in the
 * reference's rows).  rows: host array, n_rows in 1..256, each in [0, T);
 * out [B][n_head][n_rows][T] contiguous. */
int wha_wave_probs_rows(const wha_wave_cache* cache, const wha_wave_shape* shape, const int32_t* rows,
                        int32_t n_rows, float* out, void* stream);

/* Kernel family of wha_wave_fwd / wha_wave_bwd, process-wide (no counterpart
 * in the reference; for tests and benchmarks).  mode 1 = bucket-sparse: every
 * (b,h)'s positions sorted by bucket, scores computed only in the 16 x 16
 * blocks the bucket mask can admit, the previous-position term added per
 * query; 0 = every causal pair scored and the mask applied per score;
 * 2 (the default) = bucket-sparse for T >= 1024, where it is measured no
 * slower, all pairs below.  Both give the reference's results within fp32
 * rounding; the sparse family needs up to twice the score-gradient workspace,
 * which wha_wave_bwd_workspace_size always includes.  Returns the previous
 * mode, or -1 (mode unchanged) for a mode outside 0..2. */
int wha_wave_set_bucket_sparse(int mode);

/* Host forms (one sequence, host arrays, synchronous), for callers that keep
 * activations on the host as the reference does.  `w` holds HOST pointers in
 * the wha_wave_weights layout; x, out, d_attn_out, d_x are [T][n_embd].
 *
 * wave_attention_forward (attn.rs:90-305): out, and optionally the per-head
 * phases phase_out [n_head][T] (WaveAttnCache.phases). */
int wha_host_wave_attention_forward(const float* x, const wha_wave_weights* w, int32_t T, int32_t n_embd,
                                    int32_t n_head, int32_t content_dim, float* out, float* phase_out);

/* wave_attention_backward_full (attn.rs:346-430), or _pathway (:432-511) when
 * every weight-gradient pointer of `g` is NULL.  The forward intermediates are
 * recomputed on the device from x and w (the reference passes its cache).
 * `g` holds HOST pointers in the wha_wave_grads layout. */
int wha_host_wave_attention_backward(const float* x, const float* d_attn_out, const wha_wave_weights* w,
                                     int32_t T, int32_t n_embd, int32_t n_head, int32_t content_dim,
                                     const wha_wave_grads* g);

/* ---------------------------------------------------------------- wave KV cache
 * Serving (src/common/kv_cache.rs:93-356, driven by
 * src/serve_tier/inference.rs:29-106): the attention half of prefill and
 * forward_one for B concurrent sequences.  Like the reference's cache path,
 * these score phases only (no content bias, kv_cache.rs:150-162, :285-298)
 * even when the weights carry a content projection.
 *
 * Cache of one layer (HeadCache, kv_cache.rs:35-41), caller-allocated device
 * buffers with room for `capacity` positions per (sequence, head):
 *   cs     [B][n_head][capacity][2]         cos(n phi), sin(n phi)
 *   bucket [B][n_head][capacity]            phase_to_bucket(phi)
 *   phase  [B][n_head][capacity]            phi
 *   values [B][n_head][capacity][head_dim]  value rows (16-byte aligned) */
typedef struct wha_wave_kv_cache {
  float* cs;
  int32_t* bucket;
  float* phase;
  float* values;
  int32_t capacity;
} wha_wave_kv_cache;

/* Workspace bytes of wha_wave_kv_prefill for prompts of shape->T positions. */
size_t wha_wave_kv_prefill_workspace_size(const wha_wave_shape* shape);

/* prefill's attention (kv_cache.rs:121-193) over prompts x [B][T][n_embd]
 * (shape->T <= capacity): out [B][T][n_embd] after out_proj, and cache entries
 * for positions 0 .. T-1 of every sequence. */
int wha_wave_kv_prefill(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape,
                        const wha_wave_kv_cache* kv, float* out, void* workspace, size_t workspace_bytes,
                        void* stream);

/* Workspace bytes of wha_wave_kv_decode for shape->B sequences and caches of
 * up to `capacity` positions. */
size_t wha_wave_kv_decode_workspace_size(const wha_wave_shape* shape, int32_t capacity);

/* forward_one's attention (kv_cache.rs:263-335) for one new token per
 * sequence: x [B][n_embd] (shape->T must be 1), lengths = host array of the B
 * cached lengths (each in [0, capacity - 1]; B <= 256).  Writes out [B][n_embd]
 * after out_proj and appends each new position at index lengths[b]; the
 * caller then advances its lengths (cache.n_cached += 1, :358). */
int wha_wave_kv_decode(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape,
                       const wha_wave_kv_cache* kv, const int32_t* lengths, float* out, void* workspace,
                       size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- inputs
 * Seeded synthetic inputs (host): continues the xorshift64 stream in *state
 * (the reference's Rng::next_u64/next_f32, src/common/rng.rs:24-34) with
 * Box-Muller normals times stddev, and advances *state.  Multi-threaded by
 * jumping ahead in the stream; output identical to the sequential stream.
 * nthreads <= 0 picks a default.  Returns 0, or -1 for a zero state. */
int wha_synth_normal(uint64_t* state, float* out, size_t n, double stddev, int nthreads);

/* ---------------------------------------------------------------- timing
 * Optional per-kernel timing with HIP events recorded on the launch stream
 * around every kernel the library enqueues (off by default).  Used by the
 * benchmark to measure each kernel's average duration live. */
int wha_timing_enable(int on);
int wha_timing_reset(void);
/* Synchronises the recorded events and returns the summed duration (ms) and
 * launch count of the named kernel ("attn_fwd", "attn_bwd_dq", "attn_bwd_dkv",
 * "attn_bwd_delta", "decode_split", "decode_merge", ...). */
int wha_timing_read(const char* kernel, double* total_ms, int64_t* launches);

#ifdef __cplusplus
}
#endif
#endif /* WAVE_HIP_ATTN_H */
