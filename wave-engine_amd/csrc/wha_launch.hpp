// Host-side launch interface between the C ABI (wha_api.hip) and the kernel
// translation units.  Each launcher validates nothing (wha_api.hip does), picks
// the template instance for the padded head dimension and vector mode, and
// enqueues on `stream`.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "wha_device.hpp"

namespace wha {

// Feature width of the wave-attention score contraction (cos, sin, content, zero pad).
constexpr int kWaveFeatures = 32;

// Padded head dimension used by the kernels for a given D (0 = unsupported).
inline int padded_dim(int D) {
  if (D <= 0) return 0;
  if (D <= 48) return 48;
  if (D <= 64) return 64;
  if (D <= 128) return 128;
  return 0;
}

// Head dims the direct-to-LDS kernels serve (with 128-bit operands): 48, 64
// and 128, and 36..44 / 52..60 / 68..124 on the 48- / 64- / 128-wide kernels
// with the LDS quads past D fetched as zeros (those pad the same way in the
// register-staged kernels).
inline bool dma_head_dim(int D) { return D % 4 == 0 && D > 32 && D <= 128; }

// Head dims of the kept-scores pair: the same.
inline bool kept_head_dim(int D) { return dma_head_dim(D); }

// The direct-to-LDS backward reaches one head's dS (and kept scores) through
// buffer descriptors, whose byte ranges are 31-bit here: up to T of about 30000.
inline bool ds_head_fits(const View& L) { return ds_rows(L.T) * 256 < ((int64_t)1 << 31); }

// Small problems -- fewer than kSmallBlocks 64-row tiles over all (b,h) heads
// and rows of at most kSmallMaxT -- run the 16-row split-sweep kernels of
// attn_small.hip (wha_attn_fwd / wha_attn_bwd; such layouts keep no scores).
constexpr int kSmallBlocks = 256;
constexpr int kSmallMaxT = 1024;
bool small_problem(const View& L);

// Block-to-tile mapping of the direct-to-LDS kernels: by default a block takes
// the 64-row tiles p and n-1-p of one (b,h) (equal causal work per block).
// When those ceil(n/2)*B*H blocks would not give every CU three, each block
// takes one tile instead, the longest first, so the shorter tiles fill the
// slots the longer ones leave (the 384-dim config: 1024 blocks, not 512).
inline int dma_unpaired(const View& L) {
  return (int64_t)((L.T + 63) / 64 + 1) / 2 * L.B * L.H < 3 * 256 ? 1 : 0;
}
inline int64_t dma_tiles(const View& L, int unpaired) {
  const int n = (L.T + 63) / 64;
  return unpaired ? n : (n + 1) / 2;
}

// Optional per-kernel HIP-event timing (implemented in wha_api.hip).
struct TimingScope {
  TimingScope(const char* name, hipStream_t stream);
  ~TimingScope();
  void* token;
  hipStream_t stream;
};

// Fused forward.  scores != nullptr (only where scores_kept(L, vec)): also
// writes the raw scores q.k*scale*log2(e) of the causal half into it, in the
// layout of the dS buffer (bwd_ds_floats(L) floats).
hipError_t launch_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                           const View& L, bool vec, float scale, hipStream_t stream, float* scores = nullptr);

// The small-problem kernels (attn_small.hip): forward, and the backward in one
// launch (dK and dV key-stationary, dQ query-stationary with S and dP
// recomputed; Delta formed in place; no workspace).
hipError_t launch_attn_fwd_small(const float* q, const float* k, const float* v, float* o, float* lse,
                                 const View& L, float scale, hipStream_t stream);
hipError_t launch_attn_bwd_small(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                                 const float* lse, float* dq, float* dk, float* dv, const View& L, float scale,
                                 hipStream_t stream);

// Delta pass of the from-probabilities backward on the forward's direct-to-LDS
// tiles (dma_head_dim(D), 128-bit operands): stats <- the -Delta blocks of
// attn_bwd_dkv_dma_kernel, Delta_t = sum_j att[t][j] (dO_t . V_j).  av: T % 4
// == 0 and att 16-byte aligned (128-bit att loads).
hipError_t launch_probs_delta_dma(const float* d_o, const float* v, const float* att, float* stats, const View& L,
                                  bool av, hipStream_t stream);

// Whether the forward can keep its scores for this layout (the direct-to-LDS
// kernels: 16-byte-aligned operands, kept_head_dim(D), not a small problem).
bool scores_kept(const View& L, bool vec);

// Floats of the dS buffer the fused backward uses (the causal half of the
// score matrix in 64-key column blocks, fp32).
size_t bwd_ds_floats(const View& L);

// Floats of the row-statistics scratch of the fused backward (Delta, or for
// head dim 64 the -LSE*log2(e) / -Delta blocks of attn_bwd_stats_kernel).
size_t bwd_stats_floats(const View& L);

// Fused backward: Delta pre-pass, then either (ds != nullptr) the key-stationary
// dK/dV kernel writing dS to ds and a query-stationary dQ = dS K kernel, or
// (ds == nullptr) a query-stationary dQ kernel that recomputes S and dP and the
// key-stationary dK/dV kernel.  Both deterministic.  delta: bwd_stats_floats(L)
// floats of scratch.
// scores != nullptr: the forward's kept scores (launch_attn_fwd; requires ds
// and scores_kept(L, vec)), read by the dK/dV kernel instead of recomputing S.
hipError_t launch_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                           const float* d_o, const float* lse, float* dq, float* dk, float* dv,
                           float* delta, float* ds, const View& L, bool vec, float scale,
                           hipStream_t stream, const float* scores = nullptr);

// Backward from given probabilities att [B][H][T][T].  delta: [B*H*T] scratch;
// stats: bwd_stats_floats(L) scratch (the direct-to-LDS path's -Delta blocks);
// ds: bwd_ds_floats(L) scratch for the dS tiles, or nullptr to recompute dP in
// a query-stationary dQ pass instead.
hipError_t launch_attn_bwd_probs(const float* d_o, const float* q, const float* k, const float* v,
                                 const float* att, float* dq, float* dk, float* dv, float* delta, float* stats,
                                 float* ds, const View& L, bool vec, float scale, hipStream_t stream);

// Split-K decode.  Workspace layout and size: decode_workspace_floats().
size_t decode_workspace_floats(const View& cache);
hipError_t launch_decode(const float* q, const float* kc, const float* vc, float* o, float* lse,
                         float* ws, const View& cache, bool vec, float scale, hipStream_t stream);

// Rows of P recomputed from q, k and the forward's LSE (kernel argument by value).
constexpr int kMaxProbRows = 256;
struct RowList {
  int n;
  int rows[kMaxProbRows];
};
hipError_t launch_attn_probs_rows(const float* q, const float* k, const float* lse, const RowList& rl, float* out,
                                  const View& L, float scale, hipStream_t stream);

// Projections (fp32 MFMA GEMM).  x: [M][K] rows with stride ldx, w: [N][K]
// row-major, b: [N] or nullptr, y: [M][N] rows with stride ldy.
hipError_t launch_linear_fwd(const float* x, int64_t ldx, const float* w, const float* b, float* y, int64_t ldy,
                             int M, int N, int K, hipStream_t stream);
// dx[m][k] = sum_n dy[m][n] w[n][k]
hipError_t launch_linear_bwd_dx(const float* dy, int64_t lddy, const float* w, float* dx, int64_t lddx, int M,
                                int N, int K, hipStream_t stream);
// dw[n][k] = sum_m dy[m][n] x[m][k]; db[n] = sum_m dy[m][n] (db may be nullptr).
// ws: linear_dw_workspace_floats(N, K, M) floats.
size_t linear_dw_workspace_floats(int N, int K, int64_t M);
size_t linear_dw_workspace_floats(int N, int K, int64_t M, int batch);
hipError_t launch_linear_bwd_dw(const float* dy, int64_t lddy, const float* x, int64_t ldx, float* dw, float* db,
                                int M, int N, int K, float* ws, hipStream_t stream);
// Batched forms: `batch` independent problems, operand bt offset by bt * (its _sb stride).
// ws: linear_fwd_workspace_floats floats (split-K for shapes with few output
// tiles) or nullptr (no split).
size_t linear_fwd_workspace_floats(int M, int N, int K, int batch);
hipError_t launch_linear_fwd_batched(const float* x, int64_t ldx, int64_t x_sb, const float* w, int64_t w_sb,
                                     const float* b, int64_t b_sb, float* y, int64_t ldy, int64_t y_sb, int M,
                                     int N, int K, int batch, hipStream_t stream, float* ws = nullptr);
hipError_t launch_linear_bwd_dx_batched(const float* dy, int64_t lddy, int64_t dy_sb, const float* w,
                                        int64_t w_sb, float* dx, int64_t lddx, int64_t dx_sb, int M, int N,
                                        int K, int batch, bool accumulate, hipStream_t stream);
// db: [batch][N] or nullptr; ws: linear_dw_workspace_floats(N, K, M, batch) floats.
hipError_t launch_linear_bwd_dw_batched(const float* dy, int64_t lddy, int64_t dy_sb, const float* x,
                                        int64_t ldx, int64_t x_sb, float* dw, int64_t dw_sb, float* db, int M,
                                        int N, int K, int batch, float* ws, hipStream_t stream);

// Backward building blocks shared with the wave-attention path.
// Delta[b,h,t] = sum_d dO . O over the view's head.
hipError_t launch_attn_bwd_delta(const float* o, const float* d_o, float* delta, const View& L, const char* name,
                                 hipStream_t stream);
// dQ = scale * dS K from the dS workspace (ds_block_row layout); L.D must be kWaveFeatures.
hipError_t launch_dq_from_ds(const float* k, const float* ds, float* dq, const View& L, float scale,
                             const char* name, hipStream_t stream);

// ---- wave (harmonic coherence) attention ----
// proj [B][T][H][2+C] -> feat [B][H][T][kWaveFeatures], phase, bucket [B][H][T];
// the first C_used content columns become features (0: the phase-only score).
hipError_t launch_wave_features(const float* proj, const float* hraw, float* feat, float* phase, int* bucket,
                                int B, int H, int T, int C, int C_used, hipStream_t stream);
// Fused forward over the per-head values (view Lv, D = head_dim): merged
// head outputs (same view) and natural-log LSE [B][H][T].
hipError_t launch_wave_fwd(const float* feat, const int* bucket, const float* v, float* merged, float* lse,
                           const View& Lv, bool vec, float cs, hipStream_t stream);
// Core backward: Delta, dV, raw feature gradients of the key (dfk) and query
// (dfq) roles [B][H][T][kWaveFeatures]; ds: bwd_ds_floats(Lv) floats.
hipError_t launch_wave_bwd_core(const float* feat, const int* bucket, const float* v, const float* merged,
                                const float* d_merged, const float* lse, float* delta, float* dfk, float* dfq,
                                float* dv, float* ds, const View& Lv, bool vec, float cs, hipStream_t stream);

// Bucket-sparse wave attention core (wave_sparse.hip): sorts every (b,h)'s
// positions by bucket into ws and executes only the 16 x 16 blocks the bucket
// mask can admit.  ws: wave_sparse_fwd_floats (forward) or
// wave_sparse_bwd_floats (backward) floats, 16-byte aligned; ds:
// wave_sparse_ds_floats floats.
size_t wave_sparse_fwd_floats(int B, int H, int T, int D);
size_t wave_sparse_bwd_floats(int B, int H, int T, int D);
size_t wave_sparse_ds_floats(int B, int H, int T);
hipError_t launch_wave_fwd_sparse(const float* feat, const int* bucket, const float* v, float* merged, float* lse,
                                  float* ws, const View& Lv, bool vec, float cs, hipStream_t stream);
hipError_t launch_wave_bwd_core_sparse(const float* feat, const int* bucket, const float* v, const float* merged,
                                       const float* d_merged, const float* lse, float* delta, float* dfk, float* dfq,
                                       float* dv, float* ds, float* ws, const View& Lv, bool vec, float cs,
                                       hipStream_t stream);
// Rows of the wave attention probabilities: out [B][H][rl.n][T].
hipError_t launch_wave_probs_rows(const float* feat, const int* bucket, const float* lse, const RowList& rl,
                                  float* out, int B, int H, int T, float cs, hipStream_t stream);
// Feature gradients -> dproj [B][T][H][2+C]; hpart: scratch of at least B*H*T floats (per-block
// harmonic partials); d_hraw [H] or nullptr.
hipError_t launch_wave_feat_bwd(const float* proj, const float* feat, const float* phase, const float* dfq,
                                const float* dfk, const float* hraw, float* dproj, float* hpart, float* d_hraw,
                                int B, int H, int T, int C, float cs, hipStream_t stream);

// ---- wave attention KV cache (serving) ----
constexpr int kMaxKvBatch = 256;
struct KvLens {  // cached positions per sequence (kernel argument by value)
  int n;
  int len[kMaxKvBatch];
};
int wave_kv_chunk(int max_len);
size_t wave_kv_decode_part_floats(int BH, int hd, int max_len);
// Cache entries of positions [0, T) from a prompt's forward intermediates.
hipError_t launch_wave_kv_write(const float* feat, const int* bucket, const float* phase, const float* values,
                                float* cs, int* bk, float* ph, float* vc, int B, int H, int T, int hd, int E,
                                int cap, hipStream_t stream);
// One decode step: proj [B][H][2+C], vnew [B][E] -> merged [B][E]; appends at lengths[b].
// qinfo: [B*H*4] scratch, part: wave_kv_decode_part_floats(B*H, hd, max_len) scratch.
hipError_t launch_wave_kv_decode(const float* proj, const float* hraw, const float* vnew, float* merged, float* cs,
                                 int* bk, float* ph, float* vc, float* qinfo, float* part, const KvLens& ll, int B,
                                 int H, int P, int hd, int E, int cap, int max_len, bool vec, hipStream_t stream);

}  // namespace wha
