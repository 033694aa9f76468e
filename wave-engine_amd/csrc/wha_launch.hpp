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

// Padded head dimension used by the kernels for a given D (0 = unsupported).
inline int padded_dim(int D) {
  if (D <= 0) return 0;
  if (D <= 48) return 48;
  if (D <= 64) return 64;
  if (D <= 128) return 128;
  return 0;
}

// Optional per-kernel HIP-event timing (implemented in wha_api.hip).
struct TimingScope {
  TimingScope(const char* name, hipStream_t stream);
  ~TimingScope();
  void* token;
  hipStream_t stream;
};

hipError_t launch_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                           const View& L, bool vec, float scale, hipStream_t stream);

// Floats of the dS buffer the fused backward uses (the causal half of the
// score matrix in 64-key column blocks, fp32).
size_t bwd_ds_floats(const View& L);

// Fused backward: Delta pre-pass, then either (ds != nullptr) the key-stationary
// dK/dV kernel writing dS to ds and a query-stationary dQ = dS K kernel, or
// (ds == nullptr) a query-stationary dQ kernel that recomputes S and dP and the
// key-stationary dK/dV kernel.  Both deterministic.  delta: [B*H*T] scratch.
hipError_t launch_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                           const float* d_o, const float* lse, float* dq, float* dk, float* dv,
                           float* delta, float* ds, const View& L, bool vec, float scale,
                           hipStream_t stream);

// Backward from given probabilities att [B][H][T][T].  delta: [B*H*T] scratch.
hipError_t launch_attn_bwd_probs(const float* d_o, const float* q, const float* k, const float* v,
                                 const float* att, float* dq, float* dk, float* dv, float* delta,
                                 const View& L, bool vec, float scale, hipStream_t stream);

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
hipError_t launch_linear_bwd_dw(const float* dy, int64_t lddy, const float* x, int64_t ldx, float* dw, float* db,
                                int M, int N, int K, float* ws, hipStream_t stream);

}  // namespace wha
