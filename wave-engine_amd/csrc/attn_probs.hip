// On-demand export of attention-probability rows (gfx950).
//
// The fused forward never materialises P = softmax(Q K^T * scale), but the
// reference's monitors read rows of it: analyze_attention takes the last row of
// every head (src/monitors/attn_monitor.rs:26-80) and the softmax_rows value
// contract checks rows in [0, 1] summing to 1
// (src/monitors/junctions/value_range.rs:117-121).  This kernel recomputes any
// requested rows from Q, K and the forward's row log-sum-exp:
//   out[b][h][r][j] = exp(q_t . k_j * scale - lse[b][h][t])  for j <= t = rows[r], else 0.
// Rows are few (monitor use), so the kernel favours simplicity: one block per
// (b*h, row) -- b*h on grid.x, whose limit (2^31 - 1) covers every layout the
// C ABI accepts, the <= 256 rows on grid.y -- the query row in LDS, one key per
// thread per pass.
#include "wha_launch.hpp"

namespace wha {

template <int DP>
__global__ __launch_bounds__(256) void attn_probs_rows_kernel(const float* __restrict__ Q,
                                                              const float* __restrict__ K,
                                                              const float* __restrict__ LSE, RowList rl,
                                                              float* __restrict__ out, View L, float scale) {
  __shared__ float qs[DP];
  const int bh = blockIdx.x;
  const int r = blockIdx.y;
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int t = rl.rows[r];  // validated on the host: 0 <= t < T
  float* dst = out + ((int64_t)bh * rl.n + r) * L.T;
  for (int d = threadIdx.x; d < DP; d += blockDim.x) qs[d] = d < L.D ? Q[base + (int64_t)t * L.st + d] : 0.f;
  __syncthreads();
  const float lse = LSE[(int64_t)bh * L.T + t];
  for (int j = threadIdx.x; j < L.T; j += blockDim.x) {
    float p = 0.f;
    if (j <= t) {
      const float* kr = K + base + (int64_t)j * L.st;
      float dot = 0.f;
      for (int d = 0; d < L.D; ++d) dot += qs[d] * kr[d];
      p = expf(fmaf(dot, scale, -lse));  // fused: the score is not rounded before the subtraction
    }
    dst[j] = p;
  }
}

hipError_t launch_attn_probs_rows(const float* q, const float* k, const float* lse, const RowList& rl, float* out,
                                  const View& L, float scale, hipStream_t stream) {
  const dim3 grid((unsigned)(L.B * L.H), (unsigned)rl.n);
  TimingScope ts("attn_probs_rows", stream);
  switch (padded_dim(L.D)) {
    case 48:
      hipLaunchKernelGGL(attn_probs_rows_kernel<48>, grid, dim3(256), 0, stream, q, k, lse, rl, out, L, scale);
      break;
    case 64:
      hipLaunchKernelGGL(attn_probs_rows_kernel<64>, grid, dim3(256), 0, stream, q, k, lse, rl, out, L, scale);
      break;
    case 128:
      hipLaunchKernelGGL(attn_probs_rows_kernel<128>, grid, dim3(256), 0, stream, q, k, lse, rl, out, L, scale);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace wha
