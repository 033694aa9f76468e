// Fused causal attention forward for gfx950 (fp32 MFMA, online softmax).
//
// Computes, per (b,h) and query t, the same quantity as the core of
// attention_cpu (reference src/common/compute.rs:377-409):
//   o[t] = sum_{j<=t} softmax_j(q_t . k_j * scale) v_j
// without materialising the T x T score matrix, plus the row log-sum-exp the
// fused backward uses to recompute the probabilities.
//
// Work decomposition
//   block  = NW waves = 16*NW consecutive queries of one (b,h); grid = B*H*n_qtiles,
//            heaviest query tiles first; with B*H a multiple of 8 every block of
//            one (b,h) lands on the same XCD (blocks are dealt round-robin to
//            the 8 XCDs), so K/V of a head stay in that XCD's L2.
//   wave   = 16 queries.  Q lives in registers as the MFMA B operand, pre-scaled
//            by scale*log2(e) so the softmax runs in the exp2 domain.
//   K/V    = 64-key tiles staged through LDS (128-bit global loads, register
//            prefetch of the next tile while the current one is consumed).
// Per tile a wave forms S^T = K Q^T (keys on MFMA rows, its 16 queries on
// columns).  That layout leaves every lane with one query, so the running max
// needs only two cross-lane steps (VALU lane swaps), the running sum stays
// lane-local until the end, and the probabilities are already in the B-operand layout of
// O^T += V^T P^T -- no transpose through LDS.
#include "wha_launch.hpp"

namespace wha {

template <int DP, int NW, bool VEC>
__global__ __launch_bounds__(NW * 64) void attn_fwd_kernel(const float* __restrict__ Q,
                                                           const float* __restrict__ K,
                                                           const float* __restrict__ V,
                                                           float* __restrict__ O,
                                                           float* __restrict__ LSE, View L,
                                                           float scale_log2) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 16;   // queries per block
  constexpr int BN = 64;        // keys per tile
  constexpr int LD = Lds<DP>::PITCH;  // LDS row pitch (floats)
  constexpr int DG = DP / 4;    // head-dim slice per lane group
  constexpr int NDT = DP / 16;  // 16-row d tiles of O^T (row m of tile dt is d = NDT*m + dt)
  constexpr int NKT = BN / 16;  // 16-key sub-tiles of a tile
  __shared__ __align__(16) float Ks[BN * LD];
  __shared__ __align__(16) float Vs[BN * LD];

  const int BH = L.B * L.H;
  const int n_qt = (L.T + BM - 1) / BM;
  const int bh = blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int q0 = qt * BM + wave * 16;  // first query of this wave
  const int qrow = q0 + lq;            // this lane's query

  float qf[DG];
  load_row_frag<DP, VEC>(Q + base, qrow, L.T, L.D, L.st, g, scale_log2, qf);

  const int q_hi = min(L.T, (qt + 1) * BM);
  const int n_kt = (q_hi + BN - 1) / BN;

  TileStage<DP, BN, NT, VEC> ks, vs;
  ks.load(K + base, 0, L.T, L.D, L.st, tid);
  vs.load(V + base, 0, L.T, L.D, L.st, tid);

  float m_i = -INFINITY, l_i = 0.f;
  floatx4 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < n_kt; ++kt) {
    __syncthreads();
    ks.store_tile(Ks, tid);
    vs.store_tile(Vs, tid);
    __syncthreads();
    if (kt + 1 < n_kt) {
      ks.load(K + base, (kt + 1) * BN, L.T, L.D, L.st, tid);
      vs.load(V + base, (kt + 1) * BN, L.T, L.D, L.st, tid);
    }
    const int key0 = kt * BN;
    if (key0 > q0 + 15) continue;  // every key of the tile is after every query of the wave

    // S^T[key][query] (already in log2 units); four independent accumulator chains
    floatx4 s[NKT];
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) s[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
      float4 a[NKT];
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt)
        a[mt] = lds_read_quad<DP>(Ks, 16 * mt + lq, g * (DG / 4) + j);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].x, qf[4 * j + 0], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].y, qf[4 * j + 1], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].z, qf[4 * j + 2], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].w, qf[4 * j + 3], s[mt]);
    }

    // causal / tail mask, running max (one query per lane; keys over 16 values
    // in the lane and the 4 lane groups)
    // keys above key_lim are masked: one compare and a select per score, no branch
    const int key_lim = min(qrow, L.T - 1) - key0;
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float x = (16 * mt + 4 * g + i > key_lim) ? -INFINITY : s[mt][i];
        s[mt][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = pair_max32(pair_max16(mx));
    const float m_new = fmaxf(m_i, mx);
    const float alpha = fast_exp2(m_i - m_new);
    float rs = 0.f;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(s[mt][i] - m_new);
        s[mt][i] = p;
        rs += p;
      }
    }
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;

    // O^T[d][query] += V^T[d][key] P^T[key][query]; MFMA k-index g <-> key 16*mt + 4*g + i,
    // MFMA row m of d-tile dt <-> d = NDT*m + dt (one LDS read feeds all d-tiles)
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float va[NDT];
        lds_read_seg<DP, NDT>(Vs, 16 * mt + 4 * g + i, lq, va);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma4(va[dt], s[mt][i], oacc[dt]);
      }
    }
  }

  const float l_sum = pair_sum32(pair_sum16(l_i));
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] / l_sum;
  }
  store_row_frag<DP, VEC>(O + base, qrow, L.T, L.D, L.st, g, oacc, 1.f);
  if (LSE != nullptr && g == 0 && qrow < L.T)
    LSE[(int64_t)bh * L.T + qrow] = (m_i + log2f(l_sum)) * kLn2;
}

template <int DP, int NW, bool VEC>
static hipError_t launch_fwd_t(const float* q, const float* k, const float* v, float* o, float* lse,
                               const View& L, float scale, hipStream_t stream) {
  const int BM = NW * 16;
  const int n_qt = (L.T + BM - 1) / BM;
  const unsigned grid = (unsigned)(n_qt * L.B * L.H);
  const float scale_log2 = (float)((double)scale * 1.4426950408889634);
  TimingScope ts("attn_fwd", stream);
  hipLaunchKernelGGL((attn_fwd_kernel<DP, NW, VEC>), dim3(grid), dim3(NW * 64), 0, stream, q, k, v, o,
                     lse, L, scale_log2);
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                           const View& L, bool vec, float scale, hipStream_t stream) {
  switch (padded_dim(L.D)) {
    case 48:
      return vec ? launch_fwd_t<48, 4, true>(q, k, v, o, lse, L, scale, stream)
                 : launch_fwd_t<48, 4, false>(q, k, v, o, lse, L, scale, stream);
    case 64:
      return vec ? launch_fwd_t<64, 4, true>(q, k, v, o, lse, L, scale, stream)
                 : launch_fwd_t<64, 4, false>(q, k, v, o, lse, L, scale, stream);
    case 128:
      return vec ? launch_fwd_t<128, 4, true>(q, k, v, o, lse, L, scale, stream)
                 : launch_fwd_t<128, 4, false>(q, k, v, o, lse, L, scale, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace wha
