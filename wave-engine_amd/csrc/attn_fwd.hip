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
#include <type_traits>

#include "wha_launch.hpp"

#ifndef WHA_FWD_DMA
#define WHA_FWD_DMA 1
#endif


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
  // wave index as a scalar: conditions derived from it compile to scalar
  // branches, never to EXEC-masked blocks (which MFMAs would not respect)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
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

  // Running max m_i, started from an anchor (this query's score against key
  // 0, the first key of the sweep) and moved only by exact steps.  Every
  // tile's S accumulators start from -m_i, so the fused multiply-add chain of
  // the MFMA keeps its partial sums near 0 instead of rounding scores of tens
  // of units at every step (the backward, started from -LSE, then sees the
  // probabilities this forward normalised).
  float m_i, l_i = 0.f;
  {
    float kfa[DG];
    load_row_frag<DP, VEC>(K + base, 0, L.T, L.D, L.st, g, 1.f, kfa);
    float a = 0.f;
#pragma unroll
    for (int t = 0; t < DG; ++t) a = fmaf(qf[t], kfa[t], a);
    m_i = pair_sum32(pair_sum16(a));  // identical in the query's four lane groups
  }
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

    // S^T[key][query] - m_i (log2 units); four independent accumulator chains
    floatx4 s[NKT];
    // causal / tail mask: keys above key_lim, one compare and a select per
    // score, no branch
    const int key_lim = min(qrow, L.T - 1) - key0;
    auto scores = [&]() {
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = floatx4{-m_i, -m_i, -m_i, -m_i};
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
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[mt][i] = (16 * mt + 4 * g + i > key_lim) ? -INFINITY : s[mt][i];
      }
    };
    // Running max (one query per lane; keys over 16 values in the lane and
    // the 4 lane groups).  Every lane has a valid key here (key0 <= q0), so
    // mx is finite; the first tile holds the anchor's key, so there mx >= 0.
    // Scores far above the maximum they started from were summed at their
    // own size: then the tile's scores are formed again from the new maximum
    // (a second trip, whose scores are all <= 0; a loop rather than a second
    // copy of the contraction, which would hold more registers).
    float alpha = 1.f, dd;
    for (;;) {
      scores();
      float mx = -INFINITY;
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[mt][i]);
      }
      const bool redo = __builtin_amdgcn_ballot_w64(mx > kRedoMax) != 0;
      mx = pair_max32(pair_max16(mx));
      const float m_new = m_i + fmaxf(mx, 0.f);
      dd = m_new - m_i;  // exact step of the float maximum
      alpha *= fast_exp2(-dd);
      if (!redo) break;
      m_i = m_new;
    }
    const float m_new = m_i + dd;
    float rs = 0.f;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float p = fast_exp2(s[mt][i] - dd);
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

// Forward for head dims 36..128 (multiples of 4, 128-bit-aligned operands; 48,
// 64 and 128 exact, others padded up to them), arranged like the backward's
// direct-to-LDS kernels because on gfx950 every VALU instruction costs MFMA
// issue time:
//   - 32-key sub-tiles of K and V (16-key at DP = 128) go from global memory
//     straight into LDS (global_load_lds, swizzled Lds<DP> layout, two slots
//     in separate arrays, loop unrolled by two, one barrier per sub-tile,
//     per-lane fetch offsets computed once);
//   - masking runs only on sub-tiles that reach past a query of the wave or
//     past T (a wave-uniform test, separate code);
//   - the running max is refreshed, and O and the row sum rescaled, only when
//     some lane's max grew by more than kLazyMax (log2 units; a wave-uniform
//     ballot): until then the probabilities are taken against the older,
//     smaller max, so they stay below 2^kLazyMax and the fp32 sums cannot
//     overflow.  The result is the same softmax, rounded differently.
// A block handles query tiles p and n_qt-1-p (n_qt+1 key tiles of work for
// every block); grid = B*H*ceil(n_qt/2).
// SAVE: also keep the raw scores q.k*scale*log2(e) of every sub-tile it
// computes in SC (the layout of the backward's dS workspace, ds_block_row), the
// way the reference's forward hands its attention weights to the backward
// (src/common/compute.rs:391-399 -> :286-314): the key-stationary backward then
// reads them instead of recomputing Q K^T.  Entries after the diagonal hold
// whatever the key tile gave (the backward masks them); rows past T are
// written too (the layout pads every block to a multiple of 64 rows).  A
// sub-tile whose scores are formed again (see the rescale below) is stored
// again.
// DELTA: the Delta pass of the from-probabilities backward on the same tiles:
// Q is dO, K is V (scale 1), so the score contraction forms dP^T; each lane
// takes sum_j att[q][j] dP[q][j] over its keys (att given, read one sub-tile
// ahead as 16-byte loads along the row, masked entries selected away), and the
// row's -Delta goes into the stats blocks of attn_bwd_dkv_dma_kernel (LSE
// argument; 0 in the -LSE half and past T).  No softmax, no V operand, no O.
constexpr float kLazyMax = 8.f;
#ifndef WHA_FWD_WPE
#define WHA_FWD_WPE __attribute__((amdgpu_waves_per_eu(3)))
#endif
template <int DP, bool PADQ, bool SAVE, bool DELTA = false, bool AV = false>
__global__ __launch_bounds__(256) WHA_FWD_WPE void attn_fwd_dma_kernel(const float* __restrict__ Q,
                                                                     const float* __restrict__ K,
                                                                     const float* __restrict__ V,
                                                                     float* __restrict__ O,
                                                                     float* __restrict__ LSE,
                                                                     float* __restrict__ SC, View L,
                                                                     int unpaired, float scale_log2,
                                                                     const float* __restrict__ ATT = nullptr) {
  constexpr int DG = DP / 4, NDT = DP / 16;
  constexpr int QPR = DP / 4;                      // quads per row
  constexpr int BSUB = DP == 48 ? 32 : 2048 / DP;  // keys per sub-tile (8 KB per operand; 6 KB at 48)
  constexpr int NKT = BSUB / 16;                   // 16-key groups per sub-tile
  constexpr int TILE = BSUB * DP;                  // floats per operand sub-tile
  // 64-quad DMA chunks per operand sub-tile: 8 (each wave fetches two of K
  // and two of V) or, at DP = 48, 6 (waves 0-1 fetch K, waves 2-3 V, three each)
  constexpr int CH = BSUB * QPR / 64;
  constexpr bool SPLIT = CH == 6;
  constexpr int NU = SPLIT ? 3 : 2;                // chunks per wave and operand it fetches
  using LT = Lds<DP, true>;
  static_assert((CH == 8 || SPLIT) && LT::SWZ, "sub-tiles of 512 or 384 quads in the swizzled unpadded layout");
  // MFMA A-operand row m <-> tile row arow(m) (dma48_row; the Delta pass keeps
  // rows in order: its att loads want four consecutive keys per lane)
  auto arow = [](int m) { return DELTA ? m : dma48_row<DP>(m); };
  __shared__ __align__(16) float Ks0[TILE], Ks1[TILE];
  __shared__ __align__(16) float Vs0[TILE], Vs1[TILE];

  const int BH = L.B * L.H;
  const int bh = blockIdx.x % BH;
  const int pair = (int)(blockIdx.x / BH);
  const int n_qt = (L.T + 63) / 64;
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const char* kg = reinterpret_cast<const char*>(K + base);
  const char* vg = reinterpret_cast<const char*>(V + base);
  const int64_t sub_bytes = (int64_t)BSUB * L.st * 4;
  // SAVE: this head's block of the score layout as a buffer
  const __amdgpu_buffer_rsrc_t rsc =
      buffer_rsrc(SAVE ? SC + (int64_t)bh * ds_rows(L.T) * 64 : SC, SAVE ? (uint32_t)(ds_rows(L.T) * 256) : 0u);

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;

  // this lane's fetch: wave w fills LDS chunk ch(u) = 2w+u of K and V (u < 2),
  // or at DP = 48 chunk 3(w&1)+u (u < 3) of K (w < 2) or of V (w >= 2): quad
  // p = 64 ch + lane is row p / QPR, stored position p % QPR <- logical quad
  // pq_inv(row, p % QPR); byte offsets from the sub-tile's first row
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const bool v_half = SPLIT && wv >= 2;  // wave-uniform: this wave fetches V
  int rrow[NU], rcol[NU];
  uint32_t roff[NU];
  bool pad[NU];  // PADQ: this lane's quad lies past the head dim (fetched from g_zero_quad)
  auto chunk = [&](int u) { return SPLIT ? 3 * (wv & 1) + u : 2 * wv + u; };
#pragma unroll
  for (int u = 0; u < NU; ++u) {
    const int p = 64 * chunk(u) + lane;
    rrow[u] = p / QPR;
    rcol[u] = LT::pq_inv(rrow[u], p % QPR);
    pad[u] = PADQ && 4 * rcol[u] >= L.D;
    roff[u] = (uint32_t)(rrow[u] * L.st + 4 * rcol[u]) * 4u;
  }
  auto fetch = [&](int st, float* Kd, float* Vd) {
    const int k0 = st * BSUB;
    const char* ks = kg + st * sub_bytes;
    const char* vs = vg + st * sub_bytes;
    uint32_t off[NU];
#pragma unroll
    for (int u = 0; u < NU; ++u) off[u] = roff[u];
    if (k0 + BSUB > L.T) {  // last sub-tile: rows past T read row T-1
#pragma unroll
      for (int u = 0; u < NU; ++u)
        off[u] = (uint32_t)((min(k0 + rrow[u], L.T - 1) - k0) * L.st + 4 * rcol[u]) * 4u;
    }
    if constexpr (SPLIT) {
      if (DELTA && v_half) return;  // the Delta pass reads no V
      const char* src = v_half ? vs : ks;
      float* dst = v_half ? Vd : Kd;
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float* sp = reinterpret_cast<const float*>(src + off[u]);
        if (PADQ && pad[u]) sp = g_zero_quad;
        dma_quad(sp, dst + 256 * chunk(u));
      }
    } else {
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        const float* kp = reinterpret_cast<const float*>(ks + off[u]);
        const float* vp = reinterpret_cast<const float*>(vs + off[u]);
        if (PADQ && pad[u]) kp = vp = g_zero_quad;
        dma_quad(kp, Kd + 256 * chunk(u));
        if constexpr (!DELTA) dma_quad(vp, Vd + 256 * chunk(u));
      }
    }
  };

  // paired: query tiles n_qt-1-p and p (equal work per block); unpaired: one
  // tile per block, the longest first (grids too small to fill every slot)
  const int n_pass = (!unpaired && n_qt - 1 - pair != pair) ? 2 : 1;
  // sub-tiles this block sweeps, and how many it has left
  auto subs_of = [&](int qt) { return (min(L.T, (qt + 1) * 64) + BSUB - 1) / BSUB; };
  const int work = subs_of(n_qt - 1 - pair) + (n_pass == 2 ? subs_of(pair) : 0);
  int left = work;
  for (int pass = 0; pass < n_pass; ++pass) {
    const int qt = pass == 0 ? n_qt - 1 - pair : pair;  // the longer row of tiles first
    const int q0 = qt * 64 + wave * 16;                  // first query of this wave
    const int qrow = q0 + lq;                            // this lane's query
    float qf[DG];
    load_row_frag_dma<DP>(Q + base, qrow, L.T, L.D, L.st, g, scale_log2, qf);
    // running max m_i (log2 units) and row sum; -m_i in every element of neg_m,
    // from which the S accumulators start (MFMA srcC), so the scores come out
    // already shifted by the running max.  The MFMA accumulates as a chain of
    // fused multiply-adds, so starting near the row's scores keeps every
    // partial sum small and its rounding fine; summed from 0, scores of tens
    // of units pick up an ulp of their own size at every step, and the
    // backward, which starts from -LSE, would then see different
    // probabilities than the forward normalised (dQ = dS K amplifies that by
    // the size of K).  The first sub-tile starts from 0 and sets m_i; when
    // its maximum is more than kRedoMax from 0 its scores are formed again
    // from that maximum.  m_i then moves only by exact steps.
    float m_i = 0.f, l_i = 0.f;
    bool fresh = true;
    floatx4 neg_m = floatx4{0.f, 0.f, 0.f, 0.f};
    floatx4 oacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int n_sub = (min(L.T, (qt + 1) * 64) + BSUB - 1) / BSUB;
    const int key_last = min(qrow, L.T - 1);  // keys above it are masked
    // SAVE: this lane's row of the score layout, less 64 rows per column block
    // (through a buffer over this head's score blocks: below 2 GiB, scores_kept)
    const int sc_lane = (qrow * 64 + 4 * g) * 4;
    // DELTA: this lane's att row (clamped into the tensor; rows past T are never stored)
    const float* att_row = DELTA ? ATT + ((int64_t)bh * L.T + min(qrow, L.T - 1)) * L.T : nullptr;
    float d_acc = 0.f;
    floatx4 atA[NKT], atB[NKT];  // DELTA: att of the even / odd sub-tiles
    auto load_att = [&](int st, floatx4 (&dst)[NKT]) {
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
        const int c = st * BSUB + 16 * mt + 4 * g;  // keys c..c+3, clamped into the row (masked past it)
        if constexpr (AV) {
          dst[mt] = *reinterpret_cast<const floatx4*>(att_row + min(c, L.T - 4));
        } else {
#pragma unroll
          for (int i = 0; i < 4; ++i) dst[mt][i] = att_row[min(c + i, L.T - 1)];
        }
      }
    };

    auto compute = [&](auto masked, int k0, const float* Ks, const float* Vs, const floatx4 (&at)[NKT]) {
      constexpr bool MASKED = decltype(masked)::value;
      // S^T[key][query] - m_i in log2 units: MFMA rows are keys 16mt + arow(lq), columns the wave's queries
      floatx4 s[NKT];
      auto scores = [&]() {
#pragma unroll
        for (int mt = 0; mt < NKT; ++mt) {
          WHA_FENCE();
#pragma unroll
          for (int j = 0; j < DG / 4; ++j) {
            const float4 a = lds_read_quad<DP, true>(Ks, 16 * mt + arow(lq), dma48_quad<DP>(g, j));
            s[mt] = mfma4(a.x, qf[4 * j + 0], j == 0 ? neg_m : s[mt]);
            s[mt] = mfma4(a.y, qf[4 * j + 1], s[mt]);
            s[mt] = mfma4(a.z, qf[4 * j + 2], s[mt]);
            s[mt] = mfma4(a.w, qf[4 * j + 3], s[mt]);
          }
        }
        WHA_FENCE();
      };
      // SAVE: the raw scores (s + m_i, before masking) of this sub-tile
      auto keep = [&]() {
        if constexpr (SAVE) {
          const int kt = k0 >> 6;
          const int sc_blk = (int)(((ds_block_row(kt, L.T) - (int64_t)64 * kt) * 64 + (k0 & 63)) * 4);
#pragma unroll
          for (int mt = 0; mt < NKT; ++mt) buffer_store_quad(rsc, s[mt] - neg_m, sc_lane, sc_blk + 64 * mt);
        }
      };
      auto mask = [&]() {
        if (MASKED) {
#pragma unroll
          for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
              s[mt][i] = (k0 + 16 * mt + arow(4 * g + i) > key_last) ? -INFINITY : s[mt][i];
          }
        }
      };
      if constexpr (DELTA) {
        scores();
        // lane element (mt,i): dP of key k0 + 16mt + 4g + i and query qrow
#pragma unroll
        for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float t = at[mt][i] * s[mt][i];
            d_acc += (MASKED && k0 + 16 * mt + 4 * g + i > key_last) ? 0.f : t;
          }
        }
        return;
      }
      // Scores more than kLazyMax above the value the accumulators started
      // from (more than kRedoMax from 0 in the first sub-tile) were summed at
      // their own size; in that (rare) case the sub-tile's scores are formed
      // again from the new maximum, so every score that carries weight comes
      // out of a chain of small partial sums.  A loop of at most two trips
      // (the second trip's scores lie at or below the new maximum) keeps one
      // copy of the contraction.  The branches are wave-uniform scalars
      // (readfirstlane of a value every lane shares, or a ballot): the MFMAs
      // they hold ignore the EXEC mask, so these blocks must never run under
      // a partial or empty one.
      for (;;) {
        scores();
        // lane element (mt,i): key k0 + 16mt + arow(4g+i) of query qrow, as s - m_i;
        // kept at column 16mt + 4g + i of the score layout, which at DP = 48
        // therefore holds the keys of each 16-column group in tr16 order
        keep();
        mask();
        // largest shifted score among this lane's keys; the query's maximum
        // (over the 4 lane groups) is formed only where it is used -- the
        // first sub-tile and a rescale -- since some lane's maximum passes
        // kLazyMax exactly when some query's does (three-input maxima only: a
        // two-input max quiets its operands first)
        float mx;
        if constexpr (NKT == 2)
          mx = vmax3(vmax3(s[0][0], s[0][1], s[0][2]), vmax3(s[0][3], s[1][0], s[1][1]),
                     vmax3(s[1][2], s[1][3], s[0][0]));
        else
          mx = vmax3(vmax3(s[0][0], s[0][1], s[0][2]), s[0][3], s[0][0]);
        if (__builtin_amdgcn_readfirstlane((int)fresh)) {
          // first sub-tile: the running max is this one's (k0 <= every query
          // here, so every lane has a finite score)
          asm volatile("" ::: "memory");
          fresh = false;
          mx = pair_max32(pair_max16(mx));
          m_i = mx;
          neg_m = floatx4{-m_i, -m_i, -m_i, -m_i};
          if (__builtin_amdgcn_ballot_w64(fabsf(mx) > kRedoMax) != 0) continue;
#pragma unroll
          for (int mt = 0; mt < NKT; ++mt) s[mt] -= mx;
        } else if (__builtin_amdgcn_ballot_w64(mx > kLazyMax) != 0) {
          // a real branch (not if-converted): rescale to the new max, by the
          // exact step between the old and the new float maximum, and form
          // the scores again from it
          asm volatile("" ::: "memory");
          mx = pair_max32(pair_max16(mx));
          const float m_new = m_i + fmaxf(mx, 0.f);
          const float alpha = fast_exp2(-(m_new - m_i));  // the max grows by this exact step
          l_i *= alpha;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
          m_i = m_new;
          neg_m = floatx4{-m_i, -m_i, -m_i, -m_i};
          continue;
        }
        break;
      }
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) s[mt][i] = fast_exp2(s[mt][i]);
      }
      if constexpr (NKT == 2)
        l_i += ((s[0][0] + s[0][1]) + (s[0][2] + s[0][3])) + ((s[1][0] + s[1][1]) + (s[1][2] + s[1][3]));
      else
        l_i += (s[0][0] + s[0][1]) + (s[0][2] + s[0][3]);

      // O^T[d][query] += V^T[d][key] P^T[key][query] (MFMA rows: the d layout of lds_read_seg)
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
        WHA_FENCE();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float va[NDT];
          lds_read_seg<DP, NDT, true>(Vs, 16 * mt + arow(4 * g + i), lq, va);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma4(va[dt], s[mt][i], oacc[dt]);
        }
      }
    };

    // one sub-tile: wait for its loads, start the next one's, then consume it
    auto step = [&](int st, int nx, const float* Ks, const float* Vs, float* Kn, float* Vn,
                    const floatx4 (&at)[NKT], floatx4 (&at_next)[NKT]) {
      wait_vmem();
      __syncthreads();  // sub-tile st is in LDS; every wave is done with the previous one
      prio_by_remaining(left--, work);
      if (nx >= 0) {  // the next sub-tile of the sweep
        fetch(nx, Kn, Vn);
        if constexpr (DELTA) load_att(nx, at_next);
      }
      const int k0 = st * BSUB;
      if (k0 > q0 + 15) return;  // every key follows every query of the wave
      if (k0 + BSUB - 1 <= q0 && k0 + BSUB <= L.T)
        compute(std::false_type{}, k0, Ks, Vs, at);
      else
        compute(std::true_type{}, k0, Ks, Vs, at);
    };

    // Sweep order: the first pass (the longer query tile) runs from key 0
    // forward, the second from its diagonal back to key 0, so the blocks of one
    // head read at most two distinct K/V sub-tiles at any time (every block in
    // its first pass the same one, every block in its second pass the same
    // other one).  The first sub-tile a wave computes always holds a key at or
    // before every query of the wave, so its running max starts finite.
    auto st_at = [&](int j) { return pass == 0 ? j : n_sub - 1 - j; };
    __syncthreads();  // the previous pass's last sub-tile has been read by every wave
    fetch(st_at(0), Ks0, Vs0);
    if constexpr (DELTA) load_att(st_at(0), atA);
    for (int j = 0; j < n_sub; j += 2) {
      step(st_at(j), j + 1 < n_sub ? st_at(j + 1) : -1, Ks0, Vs0, Ks1, Vs1, atA, atB);
      if (j + 1 < n_sub) step(st_at(j + 1), j + 2 < n_sub ? st_at(j + 2) : -1, Ks1, Vs1, Ks0, Vs0, atB, atA);
    }

    if constexpr (DELTA) {
      // -Delta of the row into its stats block (rows past T within the block get 0)
      const float delta = pair_sum32(pair_sum16(d_acc));
      const int Tb = (L.T + 31) / 32 * 32;
      if (g == 0 && qrow < Tb) {
        float* blk = LSE + ((int64_t)bh * (Tb / 32) + qrow / 32) * 64 + qrow % 32;
        blk[0] = 0.f;
        blk[32] = qrow < L.T ? -delta : 0.f;
      }
      continue;
    }

    const float l_sum = pair_sum32(pair_sum16(l_i));
    store_row_frag_split<DP>(O + base, qrow, L.T, L.D, L.st, g, oacc, 1.f / l_sum);
    if (LSE != nullptr && g == 0 && qrow < L.T) LSE[(int64_t)bh * L.T + qrow] = (m_i + log2f(l_sum)) * kLn2;
  }
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

namespace {
template <int DP, bool PADQ>
void fwd_dma_t(const float* q, const float* k, const float* v, float* o, float* lse, float* sc, const View& L,
               float scale_log2, hipStream_t stream) {
  const int unp = dma_unpaired(L);
  const dim3 grid((unsigned)(dma_tiles(L, unp) * L.B * L.H));
  if (sc != nullptr)
    hipLaunchKernelGGL((attn_fwd_dma_kernel<DP, PADQ, true>), grid, dim3(256), 0, stream, q, k, v, o, lse, sc, L, unp,
                       scale_log2);
  else
    hipLaunchKernelGGL((attn_fwd_dma_kernel<DP, PADQ, false>), grid, dim3(256), 0, stream, q, k, v, o, lse, sc, L,
                       unp, scale_log2);
}
}  // namespace

bool scores_kept(const View& L, bool vec) {
  return WHA_FWD_DMA && WHA_DKV_DMA && vec && kept_head_dim(L.D) && ds_head_fits(L) && !small_problem(L);
}

namespace {
template <int DP, bool PADQ, bool AV>
void probs_delta_t(const float* d_o, const float* v, const float* att, float* stats, const View& L,
                   hipStream_t stream) {
  const int unp = dma_unpaired(L);
  const dim3 grid((unsigned)(dma_tiles(L, unp) * L.B * L.H));
  hipLaunchKernelGGL((attn_fwd_dma_kernel<DP, PADQ, false, true, AV>), grid, dim3(256), 0, stream, d_o, v, v,
                     (float*)nullptr, stats, (float*)nullptr, L, unp, 1.f, att);
}
}  // namespace

hipError_t launch_probs_delta_dma(const float* d_o, const float* v, const float* att, float* stats, const View& L,
                                  bool av, hipStream_t stream) {
  if (!dma_head_dim(L.D)) return hipErrorInvalidValue;
#define WHA_PD(DP, PADQ)                                                 \
  (av ? probs_delta_t<DP, PADQ, true>(d_o, v, att, stats, L, stream)   \
      : probs_delta_t<DP, PADQ, false>(d_o, v, att, stats, L, stream))
  if (L.D == 48)
    WHA_PD(48, false);
  else if (L.D < 48)
    WHA_PD(48, true);
  else if (L.D == 64)
    WHA_PD(64, false);
  else if (L.D < 64)
    WHA_PD(64, true);
  else if (L.D == 128)
    WHA_PD(128, false);
  else
    WHA_PD(128, true);
#undef WHA_PD
  return hipGetLastError();
}

hipError_t launch_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                           const View& L, bool vec, float scale, hipStream_t stream, float* scores) {
  if (scores != nullptr && !scores_kept(L, vec)) return hipErrorInvalidValue;
  if (scores == nullptr && small_problem(L)) return launch_attn_fwd_small(q, k, v, o, lse, L, scale, stream);
  if (WHA_FWD_DMA && vec && (scores != nullptr ? kept_head_dim(L.D) : dma_head_dim(L.D))) {
    const float scale_log2 = (float)((double)scale * 1.4426950408889634);
    TimingScope ts("attn_fwd", stream);
    if (L.D == 48)
      fwd_dma_t<48, false>(q, k, v, o, lse, scores, L, scale_log2, stream);
    else if (L.D < 48)
      fwd_dma_t<48, true>(q, k, v, o, lse, scores, L, scale_log2, stream);
    else if (L.D == 64)
      fwd_dma_t<64, false>(q, k, v, o, lse, scores, L, scale_log2, stream);
    else if (L.D < 64)
      fwd_dma_t<64, true>(q, k, v, o, lse, scores, L, scale_log2, stream);
    else if (L.D == 128)
      fwd_dma_t<128, false>(q, k, v, o, lse, scores, L, scale_log2, stream);
    else
      fwd_dma_t<128, true>(q, k, v, o, lse, scores, L, scale_log2, stream);
    return hipGetLastError();
  }
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
