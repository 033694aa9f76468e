// Causal attention backward for gfx950 (fp32 MFMA).
//
// Math (per (b,h); P = causal softmax(Q K^T * scale), dO = upstream gradient):
//   dV = P^T dO                      dP = dO V^T
//   dS = P o (dP - Delta),  Delta_t = sum_j P_tj dP_tj  (= dO_t . O_t)
//   dQ = scale * dS K                dK = scale * dS^T Q
// which is attention_backward_single (reference src/cpu/backward.rs:313-363)
// summed over positions by CpuBackend::attention_backward
// (src/common/compute.rs:286-314).  The reference's wgpu tier splits the same
// work into attn_backward_scores (dS and dQ per query row,
// shaders/attn_backward_scores.wgsl:27-111) and attn_backward_dkv (dK, dV per
// key, shaders/attn_backward_dkv.wgsl:22-63); this file keeps that split but
// tiles both on MFMA and never materialises dS:
//   attn_bwd_delta_kernel  Delta_t = dO_t . O_t                 (fused path)
//   attn_bwd_dq_kernel     query-stationary: recompute P, dP, dS; dQ += dS K
//   attn_bwd_dkv_kernel    key-stationary:   recompute P, dP, dS; dV += P^T dO, dK += dS^T Q
// Default fused path: the key-stationary kernel also writes its dS tiles (fp32)
// to the workspace, and attn_bwd_dq_ds_kernel forms dQ = scale * dS K with one
// MFMA contraction per tile instead of recomputing S and dP (the reference's
// wgpu tier likewise hands d_score from one kernel to the other through a
// scratch buffer, src/wgpu_tier/dispatch_backward.rs:367).  dS buffer layout
// per (b,h): column block kt (keys 64kt..64kt+63) holds rows q = 64kt..Tp-1
// (Tp = T rounded up to 64), 64 floats each, blocks back to back (ds_block_row).  When that buffer
// would be too large, attn_bwd_dq_kernel recomputes S and dP instead.
// The "from probabilities" variants read P from the caller's att tensor instead
// of recomputing it (the reference contract, att used as given), and obtain
// Delta from att and dP (mode kDeltaFromProbs) because O is not an input there.
//
// Layouts: in the query-stationary kernel a wave forms S^T/dP^T with keys on
// MFMA rows and its 16 queries on columns (one query per lane, as in the
// forward), so dS^T is directly the B operand of dQ^T += K^T dS^T.  In the
// key-stationary kernel a wave keeps its 16 keys in registers and forms S/dP
// with queries on rows and its keys on columns, so P and dS are directly the B
// operands of dV^T += dO^T P and dK^T += Q^T dS.
#include <type_traits>

#include "wha_launch.hpp"

namespace wha {

enum DqMode { kFused = 0, kProbs = 1, kDeltaFromProbs = 2 };


// Delta[r] = sum_d dO[r][d] O[r][d]: a block takes 64 rows of one (b,h), 16
// lanes per row, each 16-lane group kDeltaRows consecutive rows (all loads
// issued before the sums), no 64-bit divisions per row; the 64 results leave
// through LDS as one contiguous store.  VEC: 128-bit loads (D, the strides and
// both bases 16-byte aligned, checked on the host).
constexpr int kDeltaRows = 4;
template <bool VEC>
__global__ __launch_bounds__(256) void attn_bwd_delta_kernel(const float* __restrict__ O,
                                                             const float* __restrict__ dO,
                                                             float* __restrict__ Delta, View L) {
  const int nrb = (L.T + 63) / 64;
  const int bh = (int)(blockIdx.x / nrb), t0 = 64 * (int)(blockIdx.x % nrb);
  const int b = bh / L.H, h = bh % L.H;
  const int64_t hoff = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int sub = threadIdx.x & 15, rg = threadIdx.x >> 4;
  __shared__ float del_s[64];
  float acc[kDeltaRows];
#pragma unroll
  for (int j = 0; j < kDeltaRows; ++j) {
    acc[j] = 0.f;
    const int t = t0 + rg * kDeltaRows + j;
    if (t >= L.T) continue;
    const int64_t off = hoff + (int64_t)t * L.st;
    if (VEC) {
      for (int d = 4 * sub; d < L.D; d += 64) {
        const float4 x = *reinterpret_cast<const float4*>(dO + off + d);
        const float4 y = *reinterpret_cast<const float4*>(O + off + d);
        acc[j] += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
      }
    } else {
      for (int d = sub; d < L.D; d += 16) acc[j] += dO[off + d] * O[off + d];
    }
  }
#pragma unroll
  for (int j = 0; j < kDeltaRows; ++j) {
    float a = acc[j];
    a += __shfl_xor(a, 8, 16);
    a += __shfl_xor(a, 4, 16);
    a += __shfl_xor(a, 2, 16);
    a += __shfl_xor(a, 1, 16);
    if (sub == 0) del_s[rg * kDeltaRows + j] = a;
  }
  __syncthreads();
  if (threadIdx.x < 64 && t0 + (int)threadIdx.x < L.T) Delta[(int64_t)bh * L.T + t0 + threadIdx.x] = del_s[threadIdx.x];
}

// Row statistics for attn_bwd_dkv_dma_kernel, per (b,h) in blocks of 32 rows
// (Tb = T rounded up to 32): block j holds -LSE_t*lse_mult for t = 32j..32j+31,
// then -Delta_t for the same rows (rows past T hold 0).  The key-stationary
// kernel fetches a block with one 256-byte load and starts its S and dP
// accumulators from it.  lse_mult is log2(e) when S comes in log2 units (the
// kept scores: p = exp2(acc)) and 1/scale when S is recomputed from raw Q and
// K (acc is then in dot-product units and p = exp2(acc * scale*log2(e))).
// Same 16-lanes-per-row dot product as attn_bwd_delta_kernel.
__global__ __launch_bounds__(256) void attn_bwd_stats_kernel(const float* __restrict__ O,
                                                             const float* __restrict__ dO,
                                                             const float* __restrict__ LSE,
                                                             float* __restrict__ stats, View L, float lse_mult) {
  // block: rows t0 .. t0+63 of head bh (two 32-row stats blocks); 16 lanes per
  // row, kDeltaRows consecutive rows per 16-lane group; no 64-bit divisions
  const int Tb = (L.T + 31) / 32 * 32;
  const int nrb = (Tb + 63) / 64;
  const int bh = (int)(blockIdx.x / nrb), t0 = 64 * (int)(blockIdx.x % nrb);
  const int b = bh / L.H, h = bh % L.H;
  const int64_t hoff = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int sub = threadIdx.x & 15, rg = threadIdx.x >> 4;
  __shared__ float lse_s[64], del_s[64];
  // LSE of the block's rows, requested before the dot products
  const int tl = t0 + (int)threadIdx.x;
  const float lse = (threadIdx.x < 64 && tl < L.T) ? LSE[(int64_t)bh * L.T + tl] : 0.f;
  float acc[kDeltaRows];
#pragma unroll
  for (int j = 0; j < kDeltaRows; ++j) {
    acc[j] = 0.f;
    const int t = t0 + rg * kDeltaRows + j;
    if (t >= L.T) continue;
    const int64_t off = hoff + (int64_t)t * L.st;
    for (int d = 4 * sub; d < L.D; d += 64) {
      const float4 x = *reinterpret_cast<const float4*>(dO + off + d);
      const float4 y = *reinterpret_cast<const float4*>(O + off + d);
      acc[j] += x.x * y.x + x.y * y.y + x.z * y.z + x.w * y.w;
    }
  }
#pragma unroll
  for (int j = 0; j < kDeltaRows; ++j) {
    float a = acc[j];
    a += __shfl_xor(a, 8, 16);
    a += __shfl_xor(a, 4, 16);
    a += __shfl_xor(a, 2, 16);
    a += __shfl_xor(a, 1, 16);
    if (sub == 0) del_s[rg * kDeltaRows + j] = a;
  }
  if (threadIdx.x < 64) lse_s[threadIdx.x] = lse;
  __syncthreads();
  // stats blocks t0/32 and t0/32 + 1 (if inside Tb): 32 x -LSE*log2(e), then 32 x -Delta
  if (threadIdx.x < 128) {
    const int blk = (int)threadIdx.x >> 6, half = ((int)threadIdx.x >> 5) & 1, rr = (int)threadIdx.x & 31;
    const int t = t0 + 32 * blk + rr;
    if (t0 + 32 * blk < Tb) {
      const int i = 32 * blk + rr;
      const float v = t < L.T ? (half ? -del_s[i] : -lse_s[i] * lse_mult) : 0.f;
      stats[((int64_t)bh * (Tb / 32) + t0 / 32 + blk) * 64 + 32 * half + rr] = v;
    }
  }
}

size_t bwd_stats_floats(const View& L) { return (size_t)L.B * L.H * ((L.T + 31) / 32 * 32) * 2; }

namespace {
bool delta_vec(const float* o, const float* d_o, const View& L) {
  return ((reinterpret_cast<uintptr_t>(o) | reinterpret_cast<uintptr_t>(d_o)) & 15) == 0 && L.D % 4 == 0 &&
         L.st % 4 == 0 && L.sh % 4 == 0 && L.sb % 4 == 0;
}
hipError_t delta_launch(const float* o, const float* d_o, float* delta, const View& L, hipStream_t stream) {
  const dim3 grid((unsigned)((int64_t)L.B * L.H * ((L.T + 63) / 64)));
  if (delta_vec(o, d_o, L))
    hipLaunchKernelGGL(attn_bwd_delta_kernel<true>, grid, dim3(256), 0, stream, o, d_o, delta, L);
  else
    hipLaunchKernelGGL(attn_bwd_delta_kernel<false>, grid, dim3(256), 0, stream, o, d_o, delta, L);
  return hipGetLastError();
}
}  // namespace

// Query-stationary kernel: dQ (modes kFused, kProbs) or Delta (kDeltaFromProbs).
// In the two att modes each lane's 16 probabilities of a key tile (keys
// key0+16mt+4g+0..3 of its query row) are loaded one tile ahead, as 128-bit
// loads when AV (T % 4 == 0 and att 16-byte aligned, checked on the host);
// columns are clamped into the row and masked entries are selected away, so
// the loads need no branch and never leave att.
template <int DP, int NW, bool VEC, int MODE, bool AV = false>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dq_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LSE, float* __restrict__ Delta,
    const float* __restrict__ ATT, float* __restrict__ dQ, View L, float scale, float scale_log2) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 16;
  constexpr int BN = 64;
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int DG = DP / 4;
  constexpr int NDT = DP / 16;
  constexpr int NKT = BN / 16;
  constexpr bool kNeedK = MODE != kDeltaFromProbs;
  __shared__ __align__(16) float Ks[kNeedK ? BN * LD : 4];
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
  const int q0 = qt * BM + wave * 16;
  const int qrow = q0 + lq;
  const bool row_ok = qrow < L.T;

  float qf[MODE == kFused ? DG : 1];
  if (MODE == kFused) load_row_frag<DP, VEC>(Q + base, qrow, L.T, L.D, L.st, g, scale_log2, qf);
  float of[DG];
  load_row_frag<DP, VEC>(dO + base, qrow, L.T, L.D, L.st, g, 1.f, of);
  const int64_t rix = (int64_t)bh * L.T + qrow;
  const float lse2 = (MODE == kFused && row_ok) ? LSE[rix] * kLog2e : 0.f;
  const float delta = (MODE != kDeltaFromProbs && row_ok) ? Delta[rix] : 0.f;
  const float* att_row = (MODE != kFused) ? ATT + ((int64_t)bh * L.T + (row_ok ? qrow : 0)) * L.T : nullptr;

  const int q_hi = min(L.T, (qt + 1) * BM);
  const int n_kt = (q_hi + BN - 1) / BN;

  TileStage<DP, BN, NT, VEC> ks, vs;
  if (kNeedK) ks.load(K + base, 0, L.T, L.D, L.st, tid);
  vs.load(V + base, 0, L.T, L.D, L.st, tid);
  constexpr int NA = MODE != kFused ? NKT * 4 : 1;
  float acur[NA], anext[NA];
  auto load_att = [&](int kt) {
    if (MODE == kFused) return;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
      const int c0 = kt * BN + 16 * mt + 4 * g;
      if (AV) {
        const float4 x = *reinterpret_cast<const float4*>(att_row + min(c0, L.T - 4));
        anext[4 * mt + 0] = x.x;
        anext[4 * mt + 1] = x.y;
        anext[4 * mt + 2] = x.z;
        anext[4 * mt + 3] = x.w;
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) anext[4 * mt + i] = att_row[min(c0 + i, L.T - 1)];
      }
    }
  };
  load_att(0);

  floatx4 dqacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float dsum = 0.f;

  for (int kt = 0; kt < n_kt; ++kt) {
    __syncthreads();
    if (kNeedK) ks.store_tile(Ks, tid);
    vs.store_tile(Vs, tid);
    if (MODE != kFused) {
#pragma unroll
      for (int a = 0; a < NA; ++a) acur[a] = anext[a];
    }
    __syncthreads();
    if (kt + 1 < n_kt) {
      if (kNeedK) ks.load(K + base, (kt + 1) * BN, L.T, L.D, L.st, tid);
      vs.load(V + base, (kt + 1) * BN, L.T, L.D, L.st, tid);
      load_att(kt + 1);
    }
    const int key0 = kt * BN;
    if (key0 > q0 + 15) continue;

    // S starts from -LSE*log2(e) and dP from -Delta of this lane's query, so
    // the large partial sums of S cancel in the first steps (Delta is 0 in the
    // kDeltaFromProbs pass, which needs dP itself)
    floatx4 s[NKT], dp[NKT];
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
      s[mt] = floatx4{-lse2, -lse2, -lse2, -lse2};
      dp[mt] = floatx4{-delta, -delta, -delta, -delta};
    }
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
        if (MODE == kFused) {
          const float4 a = lds_read_quad<DP>(Ks, 16 * mt + lq, g * (DG / 4) + j);
          s[mt] = mfma4(a.x, qf[4 * j + 0], s[mt]);
          s[mt] = mfma4(a.y, qf[4 * j + 1], s[mt]);
          s[mt] = mfma4(a.z, qf[4 * j + 2], s[mt]);
          s[mt] = mfma4(a.w, qf[4 * j + 3], s[mt]);
        }
        const float4 c = lds_read_quad<DP>(Vs, 16 * mt + lq, g * (DG / 4) + j);
        dp[mt] = mfma4(c.x, of[4 * j + 0], dp[mt]);
        dp[mt] = mfma4(c.y, of[4 * j + 1], dp[mt]);
        dp[mt] = mfma4(c.z, of[4 * j + 2], dp[mt]);
        dp[mt] = mfma4(c.w, of[4 * j + 3], dp[mt]);
      }
    }

    // P (recomputed or read), dS; lane element (mt,i) is key key0+16mt+4g+i of query qrow
    // keys above key_lim are masked (and every key of a row past T): compare + select
    const int key_lim = (row_ok ? min(qrow, L.T - 1) : -1) - key0;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = 16 * mt + 4 * g + i <= key_lim;
        float p;
        if (MODE == kFused) {
          p = fast_exp2(s[mt][i]);
          p = valid ? p : 0.f;
        } else {
          p = valid ? acur[4 * mt + i] : 0.f;
        }
        if (MODE == kDeltaFromProbs) {
          dsum += p * dp[mt][i];
        } else {
          dp[mt][i] = p * dp[mt][i];
        }
      }
    }

    if (MODE != kDeltaFromProbs) {
      // dQ^T[d][query] += K^T[d][key] dS^T[key][query]  (d = NDT*m + dt on MFMA rows)
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float ka[NDT];
          lds_read_seg<DP, NDT>(Ks, 16 * mt + 4 * g + i, lq, ka);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = mfma4(ka[dt], dp[mt][i], dqacc[dt]);
        }
      }
    }
  }

  if (MODE == kDeltaFromProbs) {
    dsum = pair_sum32(pair_sum16(dsum));
    if (g == 0 && row_ok) Delta[rix] = dsum;
  } else {
    store_row_frag<DP, VEC>(dQ + base, qrow, L.T, L.D, L.st, g, dqacc, scale);
  }
}

// Key-stationary kernel: dK and dV for NW*16 consecutive keys of one (b,h);
// with DS_OUT also writes the dS tiles it forms to DS (layout: ds_block_row).
template <int DP, int NW, bool VEC, bool PROBS, bool DS_OUT>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dkv_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ LSE, const float* __restrict__ Delta,
    const float* __restrict__ ATT, float* __restrict__ dK, float* __restrict__ dV,
    float* __restrict__ DS, View L, float scale, float scale_log2) {
  constexpr int NT = NW * 64;
  constexpr int BNK = NW * 16;  // keys per block
  constexpr int BMQ = 64;       // queries per tile
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int DG = DP / 4;
  constexpr int NDT = DP / 16;
  constexpr int NQT = BMQ / 16;
  static_assert(!DS_OUT || BNK == 64, "a dS column block is 64 keys wide");
  __shared__ __align__(16) float Qs[BMQ * LD];
  __shared__ __align__(16) float Os[BMQ * LD];  // dO tile
  __shared__ __align__(16) float lse_s[BMQ];
  __shared__ __align__(16) float del_s[BMQ];

  const int BH = L.B * L.H;
  const int bh = blockIdx.x % BH;
  const int kt = (int)(blockIdx.x / BH);  // kt = 0 (the most query tiles) first
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int k0w = kt * BNK + wave * 16;  // first key of this wave
  const int krow = k0w + lq;             // this lane's key

  // K unscaled: S is the plain dot product started from -LSE/scale, and
  // scale*log2(e) is applied per score in the exponent (the forward's rounding
  // of q*scale*log2(e) is common to a row's keys; a per-key rounding here
  // would not be, and dQ = dS K amplifies that mismatch by the size of K)
  float kf[PROBS ? 1 : DG];
  if (!PROBS) load_row_frag<DP, VEC>(K + base, krow, L.T, L.D, L.st, g, 1.f, kf);
  float vf[DG];
  load_row_frag<DP, VEC>(V + base, krow, L.T, L.D, L.st, g, 1.f, vf);

  floatx4 dkacc[NDT], dvacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dkacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  const int n_qt = (L.T + BMQ - 1) / BMQ;
  const int qt0 = (kt * BNK) / BMQ;
  const int64_t rbase = (int64_t)bh * L.T;

  TileStage<DP, BMQ, NT, VEC> qs, os;
  float lse_r = 0.f, del_r = 0.f;
  // PROBS: this lane's 16 entries att[q][krow] of the next query tile
  // (q = qt*BMQ + 16mt + 4g + i), loaded with the tile; row and column are
  // clamped into att and masked entries are selected away after the MFMAs
  constexpr int NA = PROBS ? NQT * 4 : 1;
  float acur[NA], anext[NA];
  const float* att_col = PROBS ? ATT + rbase * L.T + min(krow, L.T - 1) : nullptr;
  auto load_tile = [&](int qt) {
    qs.load(Q + base, qt * BMQ, L.T, L.D, L.st, tid);
    os.load(dO + base, qt * BMQ, L.T, L.D, L.st, tid);
    if (PROBS) {
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
          anext[4 * mt + i] = att_col[(int64_t)min(qt * BMQ + 16 * mt + 4 * g + i, L.T - 1) * L.T];
      }
    }
    // raw LSE (scaled when stored to LDS): arithmetic on a value here would wait
    // for its load and, with it, for the tile loads issued just before
    if (tid < BMQ) {
      const int q = qt * BMQ + tid;
      lse_r = (!PROBS && q < L.T) ? LSE[rbase + q] : 0.f;
      del_r = q < L.T ? Delta[rbase + q] : 0.f;
    }
  };
  if (qt0 < n_qt) load_tile(qt0);

  for (int qt = qt0; qt < n_qt; ++qt) {
    __syncthreads();
    qs.store_tile(Qs, tid);
    os.store_tile(Os, tid);
    if (tid < BMQ) {
      lse_s[tid] = -lse_r / scale;
      del_s[tid] = -del_r;
    }
    if (PROBS) {
#pragma unroll
      for (int a = 0; a < NA; ++a) acur[a] = anext[a];
    }
    __syncthreads();
    if (qt + 1 < n_qt) load_tile(qt + 1);
    const int qb = qt * BMQ;
    if (qb + BMQ - 1 < k0w) continue;  // every query of the tile precedes every key of the wave
    const int q_end = krow < L.T ? L.T : 0;  // valid queries: krow <= q < q_end

    // S and dP start from -LSE/scale and -Delta of their rows (lane element
    // (mt,i): query qb+16mt+4g+i), so the large partial sums of S cancel in
    // the first steps and dS = P * dP needs no subtraction
    floatx4 s[NQT], dp[NQT];
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
      s[mt] = *reinterpret_cast<const floatx4*>(&lse_s[16 * mt + 4 * g]);
      dp[mt] = *reinterpret_cast<const floatx4*>(&del_s[16 * mt + 4 * g]);
    }
    // S and dP: 2*NQT independent accumulator chains, interleaved step by step
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
      float4 a[NQT], c[NQT];
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt) {
        if (!PROBS) a[mt] = lds_read_quad<DP>(Qs, 16 * mt + lq, g * (DG / 4) + j);
        c[mt] = lds_read_quad<DP>(Os, 16 * mt + lq, g * (DG / 4) + j);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mt = 0; mt < NQT; ++mt) {
          if (!PROBS) {
            const float av[4] = {a[mt].x, a[mt].y, a[mt].z, a[mt].w};
            s[mt] = mfma4(av[e], kf[4 * j + e], s[mt]);
          }
          const float cv[4] = {c[mt].x, c[mt].y, c[mt].z, c[mt].w};
          dp[mt] = mfma4(cv[e], vf[4 * j + e], dp[mt]);
        }
      }
    }

    // lane element (mt,i): query qb+16mt+4g+i, key krow; masking is a select,
    // so no branch sits between the MFMA blocks.
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = qb + 16 * mt + 4 * g + i;
        const bool valid = (q >= krow) & (q < q_end);
        float p;
        if (!PROBS) {
          p = fast_exp2(s[mt][i] * scale_log2);
          p = valid ? p : 0.f;
        } else {
          p = valid ? acur[4 * mt + i] : 0.f;
        }
        s[mt][i] = p;
        dp[mt][i] = p * dp[mt][i];
      }
    }

    if (DS_OUT) {
      // dS[q][64kt + 16*wave + lq] for this lane's 16 queries q = qb + 16mt + 4g + i:
      // the workspace has rows up to T rounded up to 64, so the whole tile is
      // stored without per-row checks, at constant offsets from one address
      float* dsq = DS + ((int64_t)bh * ds_rows(L.T) + ds_block_row(kt, L.T) - (int64_t)64 * kt + qb + 4 * g) * 64 +
                   wave * 16 + lq;
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dsq[(16 * mt + i) * 64] = dp[mt][i];
      }
    }

    // dV^T[d][key] += dO^T[d][query] P[query][key];  dK^T[d][key] += Q^T[d][query] dS[query][key]
    // (d = NDT*m + dt on MFMA rows: one LDS read per operand row feeds all d-tiles)
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float oa[NDT], qa[NDT];
        lds_read_seg<DP, NDT>(Os, 16 * mt + 4 * g + i, lq, oa);
        lds_read_seg<DP, NDT>(Qs, 16 * mt + 4 * g + i, lq, qa);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dvacc[dt] = mfma4(oa[dt], s[mt][i], dvacc[dt]);
          dkacc[dt] = mfma4(qa[dt], dp[mt][i], dkacc[dt]);
        }
      }
    }
  }

  store_row_frag<DP, VEC>(dK + base, krow, L.T, L.D, L.st, g, dkacc, scale);
  store_row_frag<DP, VEC>(dV + base, krow, L.T, L.D, L.st, g, dvacc, 1.f);
}

// Key-stationary dK/dV (and dS) for head dims 48, 64 and 128 (and those padded
// up to them) with 128-bit-aligned operands: the contractions of
// attn_bwd_dkv_kernel<DP, 4, true, false, DS_OUT>,
// arranged to keep the MFMA pipe fed.  On gfx950 every VALU instruction a SIMD
// issues costs MFMA issue time (an fp32 MFMA and a VALU op do not overlap), so
// the loop is built to need as little VALU work as possible:
//   - 32-query sub-tiles of Q and dO go from global memory straight into LDS
//     (global_load_lds), two LDS slots, one barrier per sub-tile: the next
//     sub-tile streams in while the current one is consumed, no registers hold
//     staged data, and every lane's fetch offsets are computed once (only a
//     uniform base moves per sub-tile).  The two slots are separate LDS arrays
//     and the loop is unrolled by two, so the compiler can tell the reads of
//     one slot from the loads into the other and does not wait for those loads
//     before reading;
//   - the row statistics arrive as one 256-byte block per sub-tile
//     (attn_bwd_stats_kernel: -LSE*log2(e) or -LSE/scale, then -Delta) and
//     initialise the S and dP accumulators, so P = exp2(S) (kept scores) or
//     exp2(S * scale*log2(e)) (recomputed) and dS = P * dP;
//   - masking runs only on sub-tiles that touch the diagonal or the end of the
//     sequence (a wave-uniform test);
//   - Q and dO sit in the swizzled Lds<DP> layout (a DMA instruction fills 64
//     quads of unpadded rows; lane l fetches the logical quad that belongs at
//     position l);
//   - each accumulator is one dependent MFMA chain (back-to-back accumulation
//     into the same registers issues at full rate), so S and dP of a sub-tile
//     take 8 registers each.
// Rows past T are fetched from row T-1 (in bounds) and masked.  Every dS entry
// the dQ kernel reads is stored: a wave skips a sub-tile only when all its rows
// precede the wave's keys.  A block handles key tiles p and n_kt-1-p (n_kt+1
// key-tile x query-tile products for every block), so equal blocks fill the
// CUs to the end instead of leaving a tail of short blocks;
// grid = B*H*ceil(n_kt/2).
// SAVED: S comes from the forward's kept scores SC (attn_fwd_dma_kernel with
// SAVE, same layout as DS) instead of Q K^T: a lane's 8 scores of the next
// sub-tile are loaded while the current one is consumed (two register sets,
// alternating with the unrolled loop), and K is not needed at all.
// PROBS (with SAVED): SC is the caller's att [B][H][T][T] and P is read as
// given (the reference's attention_backward contract, src/cpu/backward.rs:330):
// no exponential, rows and columns clamped into the tensor (those entries are
// masked), entries after the diagonal never used unmasked; the stats blocks
// then hold only -Delta (the Delta pass, launch_probs_delta_dma).
// three blocks per CU at head dims 48 and 64, two at 128 (LDS and VGPR budgets)
#ifndef WHA_DMA_WPE
#define WHA_DMA_WPE(DP) __attribute__((amdgpu_waves_per_eu((DP) <= 64 ? 3 : 2)))
#endif
template <int DP, bool DS_OUT, bool PADQ, bool SAVED, bool PROBS = false>
__global__ __launch_bounds__(256) WHA_DMA_WPE(DP) void attn_bwd_dkv_dma_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ dO, const float* __restrict__ stats, float* __restrict__ dK,
    float* __restrict__ dV, float* __restrict__ DS, const float* __restrict__ SC, View L, int unpaired,
    float scale, float scale_log2) {
  constexpr int DG = DP / 4, NDT = DP / 16;
  constexpr int QPR = DP / 4;            // quads per row
  constexpr int BSUB = 32;               // queries per sub-tile
  constexpr int TILE = BSUB * DP;        // floats per operand sub-tile
  // 64-quad DMA chunks per operand sub-tile: 8 or 16 (each wave fetches a
  // quarter of Q and of dO) or, at DP = 48, 6 (waves 0-1 fetch Q, waves 2-3 dO,
  // three each)
  constexpr int CH = BSUB * QPR / 64;
  constexpr bool SPLIT = CH == 6;
  constexpr int NF = SPLIT ? 3 : CH / 4;  // chunks per wave and operand it fetches
  using LT = Lds<DP, true>;
  static_assert(LT::SWZ && (SPLIT || CH % 4 == 0), "the DMA layout is the swizzled unpadded row");
  // MFMA A-operand row m <-> query row arow(m) of a 16-row group (dma48_row)
  auto arow = [](int m) { return dma48_row<DP>(m); };
  __shared__ __align__(16) float Qs0[TILE], Qs1[TILE];
  __shared__ __align__(16) float Os0[TILE], Os1[TILE];
  __shared__ __align__(16) float St0[2 * BSUB], St1[2 * BSUB];

  const int BH = L.B * L.H;
  const int bh = blockIdx.x % BH;
  const int pair = (int)(blockIdx.x / BH);
  const int n_kt = (L.T + 63) / 64;
  const int n_st = (L.T + BSUB - 1) / BSUB;
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const char* qg = reinterpret_cast<const char*>(Q + base);
  const char* og = reinterpret_cast<const char*>(dO + base);
  const float* stg = stats + (int64_t)bh * n_st * 64;
  const int64_t sub_bytes = (int64_t)BSUB * L.st * 4;  // one sub-tile of rows

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;

  // This lane's fetch: wave w fills LDS chunk ch(u) = NF*w+u of both operands
  // (u < NF), or at DP = 48 chunk 3(w&1)+u (u < 3) of Q (w < 2) or of dO
  // (w >= 2): quad p = 64 ch + lane is row p / QPR of the sub-tile, stored
  // position p % QPR, which holds logical quad pq_inv(row, p % QPR).  Byte offsets
  // from the sub-tile's first row; the last sub-tile clamps rows to T-1.
  const int wv = __builtin_amdgcn_readfirstlane(wave);
  const bool o_half = SPLIT && wv >= 2;  // wave-uniform: this wave fetches dO
  auto chunk = [&](int u) { return SPLIT ? 3 * (wv & 1) + u : NF * wv + u; };
  int rrow[NF], rcol[NF];
  uint32_t roff[NF];
  bool pad[NF];  // PADQ: this lane's quad lies past the head dim (fetched from g_zero_quad)
#pragma unroll
  for (int u = 0; u < NF; ++u) {
    const int p = 64 * chunk(u) + lane;
    rrow[u] = p / QPR;
    rcol[u] = LT::pq_inv(rrow[u], p % QPR);
    pad[u] = PADQ && 4 * rcol[u] >= L.D;
    roff[u] = (uint32_t)(rrow[u] * L.st + 4 * rcol[u]) * 4u;
  }
  auto fetch = [&](int st, float* Qd, float* Od, float* Sd) {
    const int q0 = st * BSUB;
    const char* qs = qg + st * sub_bytes;
    const char* os = og + st * sub_bytes;
    uint32_t off[NF];
#pragma unroll
    for (int u = 0; u < NF; ++u) off[u] = roff[u];
    if (q0 + BSUB > L.T) {  // last sub-tile: rows past T read row T-1
#pragma unroll
      for (int u = 0; u < NF; ++u) off[u] = (uint32_t)((min(q0 + rrow[u], L.T - 1) - q0) * L.st + 4 * rcol[u]) * 4u;
    }
    if constexpr (SPLIT) {
      const char* src = o_half ? os : qs;
      float* dst = o_half ? Od : Qd;
#pragma unroll
      for (int u = 0; u < NF; ++u) {
        const float* sp = reinterpret_cast<const float*>(src + off[u]);
        if (PADQ && pad[u]) sp = g_zero_quad;
        dma_quad(sp, dst + 256 * chunk(u));
      }
    } else {
#pragma unroll
      for (int u = 0; u < NF; ++u) {
        const float* qp = reinterpret_cast<const float*>(qs + off[u]);
        const float* op = reinterpret_cast<const float*>(os + off[u]);
        if (PADQ && pad[u]) qp = op = g_zero_quad;
        dma_quad(qp, Qd + 256 * chunk(u));
        dma_quad(op, Od + 256 * chunk(u));
      }
    }
    // stats position 16a + 4g + i holds the row 16a + arow(4g+i) (floatx4 reads below)
    if (wave == 0) dma_dword(stg + st * 64 + arow(lane), Sd);
  };

  // this head's dS (and kept scores, same layout) as buffers (below 2 GiB: ds_head_fits)
  const int64_t ds_head = (int64_t)bh * ds_rows(L.T) * 64;
  const uint32_t ds_rec = (uint32_t)(ds_rows(L.T) * 256);
  const __amdgpu_buffer_rsrc_t rds = buffer_rsrc(DS_OUT ? DS + ds_head : DS, DS_OUT ? ds_rec : 0u);
  const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(SAVED && !PROBS ? SC + ds_head : SC, SAVED && !PROBS ? ds_rec : 0u);

  // key tiles pair and n_kt-1-pair: every block does n_kt+1 tiles of work.
  // One key tile: 64 keys, wave w owns keys 64kt + 16w .. +15.
  // paired: key tiles p and n_kt-1-p; unpaired: one tile per block, the longest first
  const int n_pass = (!unpaired && n_kt - 1 - pair != pair) ? 2 : 1;
  // sub-tiles this block sweeps, and how many it has left
  const int work = (n_st - 2 * pair) + (n_pass == 2 ? n_st - 2 * (n_kt - 1 - pair) : 0);
  int left = work;
  for (int pass = 0; pass < n_pass; ++pass) {
    const int kt = pass == 0 ? pair : n_kt - 1 - pair;
    const int k0w = kt * 64 + wave * 16;
    const int krow = k0w + lq;
    // K unscaled: the recomputed S is the plain dot product q.k (started from
    // -LSE/scale), and scale*log2(e) is applied once per score in the
    // exponent.  The forward forms q*(scale*log2(e)) . k, whose rounding is
    // common to every key of a row and cancels against its LSE; scaling K
    // here instead would round each key's scores differently from the
    // forward's, and dQ = dS K amplifies such a per-key mismatch by the size
    // of K wherever large scores come from a large shared key component.
    float kf[SAVED ? 1 : DG], vf[DG];
    if constexpr (!SAVED) load_row_frag_dma<DP>(K + base, krow, L.T, L.D, L.st, g, 1.f, kf);
    load_row_frag_dma<DP>(V + base, krow, L.T, L.D, L.st, g, 1.f, vf);
    floatx4 dkacc[NDT], dvacc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
      dkacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
      dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
    const int q_end = krow < L.T ? L.T : 0;  // valid queries: krow <= q < q_end
    // this lane's key column of the dS and score layouts (key 16w + lq; at
    // DP = 48 the keys of each 16-column group sit in tr16 order)
    const int64_t kcol = ((int64_t)bh * ds_rows(L.T) + ds_block_row(kt, L.T) - (int64_t)64 * kt) * 64 + wave * 16 +
                         arow(lq);
    // dS (and kept scores) of row q0 + arow(4g + i) (i < 4) of this key tile's
    // block: buffer accesses with the uniform offset q0 * 256 and this lane's
    // fixed offset -- no per-lane address arithmetic
    int vrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) vrow[i] = (int)((kcol - ds_head) * 4) + arow(4 * g + i) * 256;
    // SAVED: a lane's scores of sub-tile st (rows 32st+16mt+arow(4g+i), this lane's key)
    auto load_sc = [&](int st, float (&dst)[8]) {
      if constexpr (PROBS) {
        const float* src = SC + (int64_t)bh * L.T * L.T + min(krow, L.T - 1);
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            dst[4 * mt + i] = src[(int64_t)min(st * BSUB + 16 * mt + arow(4 * g + i), L.T - 1) * L.T];
        }
      } else {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i)
            dst[4 * mt + i] = buffer_load_float(rsc, vrow[i], (st * BSUB + 16 * mt) * 256);
        }
      }
    };

    // one sub-tile's contractions; MASKED: the sub-tile touches the diagonal or
    // the end of the sequence (a separate copy, so the common case carries no
    // compare or select)
    auto compute = [&](auto masked, int qb, const float* Qs, const float* Os, const float* Sts,
                       const float (&sc)[8]) {
      constexpr bool MASKED = decltype(masked)::value;
      // S and dP, started from the rows' -LSE*log2(e) (kept scores) or
      // -LSE/scale (recompute) and -Delta
      floatx4 s[2], dp[2];
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        WHA_FENCE();
        s[mt] = *reinterpret_cast<const floatx4*>(&Sts[16 * mt + 4 * g]);
        dp[mt] = *reinterpret_cast<const floatx4*>(&Sts[BSUB + 16 * mt + 4 * g]);
#pragma unroll
        for (int j = 0; j < DG / 4; ++j) {
          if constexpr (!SAVED) {
            const float4 a = lds_read_quad<DP, true>(Qs, 16 * mt + arow(lq), dma48_quad<DP>(g, j));
            s[mt] = mfma4(a.x, kf[4 * j + 0], s[mt]);
            s[mt] = mfma4(a.y, kf[4 * j + 1], s[mt]);
            s[mt] = mfma4(a.z, kf[4 * j + 2], s[mt]);
            s[mt] = mfma4(a.w, kf[4 * j + 3], s[mt]);
          }
          const float4 c = lds_read_quad<DP, true>(Os, 16 * mt + arow(lq), dma48_quad<DP>(g, j));
          dp[mt] = mfma4(c.x, vf[4 * j + 0], dp[mt]);
          dp[mt] = mfma4(c.y, vf[4 * j + 1], dp[mt]);
          dp[mt] = mfma4(c.z, vf[4 * j + 2], dp[mt]);
          dp[mt] = mfma4(c.w, vf[4 * j + 3], dp[mt]);
        }
      }
      WHA_FENCE();
      if constexpr (SAVED) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) s[mt][i] = PROBS ? sc[4 * mt + i] : s[mt][i] + sc[4 * mt + i];
        }
      }
      // lane element (mt,i): query qb+16mt+arow(4g+i), key krow
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = PROBS ? s[mt][i] : fast_exp2(SAVED ? s[mt][i] : s[mt][i] * scale_log2);
          if (MASKED) {
            const int q = qb + 16 * mt + arow(4 * g + i);
            const bool valid = (q >= krow) & (q < q_end);
            s[mt][i] = valid ? p : 0.f;
            dp[mt][i] = valid ? p * dp[mt][i] : 0.f;
          } else {
            s[mt][i] = p;
            dp[mt][i] = p * dp[mt][i];
          }
        }
      }

      if (DS_OUT) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) buffer_store_float(rds, dp[mt][i], vrow[i], (qb + 16 * mt) * 256);
        }
      }

      // dV^T[d][key] += dO^T[d][query] P[query][key];  dK^T[d][key] += Q^T[d][query] dS[query][key]
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        WHA_FENCE();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float oa[NDT], qa[NDT];
          lds_read_seg<DP, NDT, true>(Os, 16 * mt + arow(4 * g + i), lq, oa);
          lds_read_seg<DP, NDT, true>(Qs, 16 * mt + arow(4 * g + i), lq, qa);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            dvacc[dt] = mfma4(oa[dt], s[mt][i], dvacc[dt]);
            dkacc[dt] = mfma4(qa[dt], dp[mt][i], dkacc[dt]);
          }
        }
      }
    };

    // one sub-tile: wait for its loads, start the next one's, then consume it
    auto step = [&](int st, int nx, const float* Qs, const float* Os, const float* Sts, float* Qn, float* On,
                    float* Sn, const float (&sc)[8], float (&sc_next)[8]) {
      wait_vmem();
      __syncthreads();  // sub-tile st is in LDS; every wave is done with the previous one
      prio_by_remaining(left--, work);
      if (nx >= 0) {  // the next sub-tile of the sweep
        fetch(nx, Qn, On, Sn);
        if constexpr (SAVED) load_sc(nx, sc_next);
      }
      const int qb = st * BSUB;
      if (qb + BSUB - 1 < k0w) return;  // every row precedes every key of the wave
      if (qb >= k0w + 15 && qb + BSUB <= L.T && k0w + 16 <= L.T)
        compute(std::false_type{}, qb, Qs, Os, Sts, sc);
      else
        compute(std::true_type{}, qb, Qs, Os, Sts, sc);
    };

    // Sweep order: the first pass (the longer key tile) runs from the last
    // sub-tile back to its diagonal, the second from its diagonal forward.  The
    // blocks of one head then read at most two distinct Q/dO sub-tiles at any
    // time (every block in its first pass the same one, every block in its
    // second pass the same other one), which stay in their XCD's L2.
    const int st0 = 2 * kt;
    const int nsub = n_st - st0;
    auto st_at = [&](int j) { return pass == 0 ? n_st - 1 - j : st0 + j; };
    float scA[8], scB[8];  // SAVED: scores of the even / odd steps
    __syncthreads();  // the previous key tile's last sub-tile has been read by every wave
    fetch(st_at(0), Qs0, Os0, St0);
    if constexpr (SAVED) load_sc(st_at(0), scA);
    for (int j = 0; j < nsub; j += 2) {
      step(st_at(j), j + 1 < nsub ? st_at(j + 1) : -1, Qs0, Os0, St0, Qs1, Os1, St1, scA, scB);
      if (j + 1 < nsub) step(st_at(j + 1), j + 2 < nsub ? st_at(j + 2) : -1, Qs1, Os1, St1, Qs0, Os0, St0, scB, scA);
    }
    store_row_frag_split<DP>(dK + base, krow, L.T, L.D, L.st, g, dkacc, scale);
    store_row_frag_split<DP>(dV + base, krow, L.T, L.D, L.st, g, dvacc, 1.f);
  }
}

// dQ = scale * dS K for head dims 48, 64 and 128 (and those padded up to them)
// with 128-bit-aligned operands, written for few VALU instructions per MFMA
// like attn_bwd_dkv_dma_kernel:
//   - 64-key K tiles go from global memory straight into LDS (global_load_lds,
//     swizzled Lds<DP> layout, two slots in separate arrays, loop unrolled by
//     two, one barrier per tile);
//   - a lane's 16 dS values of the next tile come as four 128-bit loads from
//     one address (dS rows sit at 256-byte pitch), straight into the MFMA B
//     operand (k-step (c, e) <-> column 16c + 4g + e, which holds key
//     16c + dma48_row(4g + e): the dK/dV kernel writes the keys of each
//     16-column group in tr16 order at DP = 48);
//   - one dependent accumulator chain per d-tile; 16-key chunks that lie after
//     every query of the wave are skipped (only in the diagonal tile, a
//     wave-uniform test).  Every dS entry read there was written by the
//     key-stationary pass (zeros where masked); rows past T feed only dQ rows
//     that are never stored.
// A block handles query tiles p and n_qt-1-p (n_qt+1 key tiles of work for
// every block); grid = B*H*ceil(n_qt/2).
template <int DP, bool PADQ>
__global__ __launch_bounds__(256) void attn_bwd_dq_dma_kernel(const float* __restrict__ K,
                                                              const float* __restrict__ DS,
                                                              float* __restrict__ dQ, View L, int unpaired,
                                                              float scale) {
  constexpr int NDT = DP / 16, BN = 64;
  constexpr int QPR = DP / 4;            // quads per row
  constexpr int TILE = BN * DP;
  constexpr int NF = BN * QPR / 256;     // DMA instructions per wave per tile
  static_assert(BN * QPR % 256 == 0, "a K tile is a whole number of DMA instructions per wave");
  using LT = Lds<DP, true>;
  __shared__ __align__(16) float Ks0[TILE], Ks1[TILE];

  const int BH = L.B * L.H;
  const int bh = blockIdx.x % BH;
  const int pair = (int)(blockIdx.x / BH);
  const int n_qt = (L.T + 63) / 64;
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const char* kg = reinterpret_cast<const char*>(K + base);
  const int64_t tile_bytes = (int64_t)BN * L.st * 4;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;

  // this lane's part of a K tile fetch: wave w fills LDS quads 64(NF*w+u) ..
  // +63 (u < NF): quad p = 64(NF*w+u) + lane is row p / QPR, stored position
  // p % QPR <- logical quad pq_inv(row, p % QPR); byte offsets from the tile's first row
  int krow_[NF], kcol[NF];
  uint32_t koff[NF];
  bool pad[NF];  // PADQ: this lane's quad lies past the head dim (fetched from g_zero_quad)
#pragma unroll
  for (int u = 0; u < NF; ++u) {
    const int p = 64 * (NF * wave + u) + lane;
    krow_[u] = p / QPR;
    kcol[u] = LT::pq_inv(krow_[u], p % QPR);
    pad[u] = PADQ && 4 * kcol[u] >= L.D;
    koff[u] = (uint32_t)(krow_[u] * L.st + 4 * kcol[u]) * 4u;
  }
  auto fetch = [&](int kt, float* Kd) {
    const char* ks = kg + kt * tile_bytes;
    if ((kt + 1) * BN > L.T) {  // last tile: rows past T read row T-1
#pragma unroll
      for (int u = 0; u < NF; ++u) {
        const uint32_t off = (uint32_t)((min(kt * BN + krow_[u], L.T - 1) - kt * BN) * L.st + 4 * kcol[u]) * 4u;
        const float* kp = reinterpret_cast<const float*>(ks + off);
        if (PADQ && pad[u]) kp = g_zero_quad;
        dma_quad(kp, Kd + 256 * (NF * wave + u));
      }
    } else {
#pragma unroll
      for (int u = 0; u < NF; ++u) {
        const float* kp = reinterpret_cast<const float*>(ks + koff[u]);
        if (PADQ && pad[u]) kp = g_zero_quad;
        dma_quad(kp, Kd + 256 * (NF * wave + u));
      }
    }
  };

  const float* dsh = DS + (int64_t)bh * ds_rows(L.T) * 64;
  // buffer loads over this head's dS (below 2 GiB: ds_head_fits)
  const __amdgpu_buffer_rsrc_t rds = buffer_rsrc(dsh, (uint32_t)(ds_rows(L.T) * 256));
  // paired: query tiles n_qt-1-p and p; unpaired: one tile per block, the longest first
  const int n_pass = (!unpaired && n_qt - 1 - pair != pair) ? 2 : 1;
  const int work = (n_qt - pair) + (n_pass == 2 ? pair + 1 : 0);  // key tiles this block sweeps
  int left = work;
  for (int pass = 0; pass < n_pass; ++pass) {
    const int qt = pass == 0 ? n_qt - 1 - pair : pair;  // the longer row of tiles first
    const int q0 = qt * 64 + wave * 16;
    const int qrow = q0 + lq;
    const int n_kt = qt + 1;
    // dS of key tile kt for this lane: row qrow of column block kt, columns
    // 16c + 4g .. +3 (the block's first row is a uniform offset)
    auto load_ds = [&](int kt, float4* dsv) {
      const int soff = (int)((ds_block_row(kt, L.T) - (int64_t)64 * kt) * 256), voff = (qrow * 64 + 4 * g) * 4;
#pragma unroll
      for (int c = 0; c < 4; ++c) dsv[c] = buffer_load_quad(rds, voff + 64 * c, soff);
    };
    floatx4 acc[NDT];
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    // dS of even tiles in dA, odd tiles in dB (the two unrolled steps swap
    // roles, so no register copies)
    float4 dA[4], dB[4];

    auto step = [&](int kt, int nx, const float* Ks, float* Kn, const float4* dcur, float4* dnext) {
      wait_vmem();
      __syncthreads();  // K tile kt is in LDS; every wave is done with the previous one
      prio_by_remaining(left--, work);
      if (nx >= 0) {  // the next tile of the sweep
        fetch(nx, Kn);
        load_ds(nx, dnext);
      }
      if (kt < qt) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          WHA_FENCE();
          const float dv[4] = {dcur[c].x, dcur[c].y, dcur[c].z, dcur[c].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float ka[NDT];
            lds_read_seg<DP, NDT, true>(Ks, 16 * c + dma48_row<DP>(4 * g + e), lq, ka);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma4(ka[dt], dv[e], acc[dt]);
          }
        }
      } else {
        // diagonal tile: chunks after every query of the wave are skipped
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          if (16 * c > wave * 16 + 15) break;
          WHA_FENCE();
          const float dv[4] = {dcur[c].x, dcur[c].y, dcur[c].z, dcur[c].w};
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float ka[NDT];
            lds_read_seg<DP, NDT, true>(Ks, 16 * c + dma48_row<DP>(4 * g + e), lq, ka);
#pragma unroll
            for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma4(ka[dt], dv[e], acc[dt]);
          }
        }
      }
    };

    // Sweep order as in the forward: the first pass from key tile 0 forward,
    // the second from its diagonal back, so the blocks of one head read at most
    // two distinct K tiles at any time.
    auto kt_at = [&](int j) { return pass == 0 ? j : n_kt - 1 - j; };
    __syncthreads();  // the previous pass's last tile has been read by every wave
    fetch(kt_at(0), Ks0);
    load_ds(kt_at(0), dA);
    for (int j = 0; j < n_kt; j += 2) {
      step(kt_at(j), j + 1 < n_kt ? kt_at(j + 1) : -1, Ks0, Ks1, dA, dB);
      if (j + 1 < n_kt) step(kt_at(j + 1), j + 2 < n_kt ? kt_at(j + 2) : -1, Ks1, Ks0, dB, dA);
    }
    store_row_frag_split<DP>(dQ + base, qrow, L.T, L.D, L.st, g, acc, scale);
  }
}

// Query-stationary dQ from stored dS: dQ^T[d][q] += K^T[d][key] dS^T[key][q] over
// the causal 64-key tiles; K tiles staged through LDS (A operand, d = NDT*m + dt
// on MFMA rows; the swizzled layout at head dim 64, where it keeps that d
// layout), dS read from the workspace with 128-bit loads straight into the
// B operand (k-step (c, e) <-> key 16c + 4g + e), one tile ahead.
template <int DP, int NW, bool VEC>
__global__ __launch_bounds__(NW * 64) void attn_bwd_dq_ds_kernel(const float* __restrict__ K,
                                                                 const float* __restrict__ DS,
                                                                 float* __restrict__ dQ, View L, float scale) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 16;
  constexpr int BN = 64;
  constexpr int LD = Lds<DP, DP == 64>::PITCH;
  constexpr int NDT = DP / 16;
  __shared__ __align__(16) float Ks[BN * LD];

  const int BH = L.B * L.H;
  const int n_qt = (L.T + BM - 1) / BM;
  const int bh = blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int q0 = qt * BM + wave * 16;
  const int qrow = q0 + lq;
  const bool row_ok = qrow < L.T;

  const float* dsh = DS + (int64_t)bh * ds_rows(L.T) * 64;
  auto load_ds = [&](int kt, float4* dsv) {
    const float* src = dsh + (ds_block_row(kt, L.T) + qrow - 64 * kt) * 64 + 4 * g;
#pragma unroll
    for (int c = 0; c < 4; ++c)
      dsv[c] = row_ok ? *reinterpret_cast<const float4*>(src + 16 * c) : make_float4(0.f, 0.f, 0.f, 0.f);
  };

  const int q_hi = min(L.T, (qt + 1) * BM);
  const int n_kt = (q_hi + BN - 1) / BN;

  TileStage<DP, BN, NT, VEC> ks;
  ks.load(K + base, 0, L.T, L.D, L.st, tid);
  float4 dcur[4], dnext[4];
  load_ds(0, dcur);

  // even and odd 16-key chunks accumulate separately: 2*NDT independent chains
  floatx4 acc[NDT], acc2[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    acc2[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }

  for (int kt = 0; kt < n_kt; ++kt) {
    __syncthreads();
    ks.template store_tile<DP == 64>(Ks, tid);
    __syncthreads();
    if (kt + 1 < n_kt) {
      ks.load(K + base, (kt + 1) * BN, L.T, L.D, L.st, tid);
      load_ds(kt + 1, dnext);
    }
#pragma unroll
    for (int c = 0; c < 4; c += 2) {
      // chunks after every query of the wave hold dS = 0 and are skipped
      const bool on0 = kt * BN + 16 * c <= q0 + 15;
      const bool on1 = kt * BN + 16 * (c + 1) <= q0 + 15;
      if (on0) {
        const float d0[4] = {dcur[c].x, dcur[c].y, dcur[c].z, dcur[c].w};
        const float d1[4] = {dcur[c + 1].x, dcur[c + 1].y, dcur[c + 1].z, dcur[c + 1].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float ka[NDT], kb[NDT];
          lds_read_seg<DP, NDT, DP == 64>(Ks, 16 * c + 4 * g + e, lq, ka);
          lds_read_seg<DP, NDT, DP == 64>(Ks, 16 * (c + 1) + 4 * g + e, lq, kb);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            acc[dt] = mfma4(ka[dt], d0[e], acc[dt]);
            acc2[dt] = mfma4(kb[dt], on1 ? d1[e] : 0.f, acc2[dt]);
          }
        }
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) dcur[c] = dnext[c];
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] += acc2[dt];
  store_row_frag<DP, VEC>(dQ + base, qrow, L.T, L.D, L.st, g, acc, scale);
}

namespace {

// Head dims dma_head_dim() accepts, 128-bit operands, dS buffer present: row
// statistics in 32-row blocks, the direct-to-LDS key-stationary kernel (dK,
// dV, dS), then dQ from dS.
template <int DP, bool PADQ>
hipError_t bwd_dma_t(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                     const float* lse, float* dq, float* dk, float* dv, float* stats, float* ds, const View& L,
                     float scale, hipStream_t stream, const float* sc) {
  const float sl2 = (float)((double)scale * 1.4426950408889634);
  const int unp = dma_unpaired(L);
  const dim3 grid((unsigned)(dma_tiles(L, unp) * L.B * L.H));
  hipError_t e;
  {
    TimingScope ts("attn_bwd_delta", stream);
    const int64_t blocks = (int64_t)L.B * L.H * (((L.T + 31) / 32 * 32 + 63) / 64);
    // kept scores are in log2 units; the recompute works in dot-product units
    const float lse_mult = sc != nullptr ? kLog2e : (float)(1.0 / (double)scale);
    hipLaunchKernelGGL(attn_bwd_stats_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, o, d_o, lse, stats, L,
                       lse_mult);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  {
    TimingScope ts("attn_bwd_dkv", stream);
    if (sc != nullptr)
      hipLaunchKernelGGL((attn_bwd_dkv_dma_kernel<DP, true, PADQ, true>), grid, dim3(256), 0, stream, q, k, v, d_o,
                         (const float*)stats, dk, dv, ds, sc, L, unp, scale, sl2);
    else
      hipLaunchKernelGGL((attn_bwd_dkv_dma_kernel<DP, true, PADQ, false>), grid, dim3(256), 0, stream, q, k, v,
                         d_o, (const float*)stats, dk, dv, ds, sc, L, unp, scale, sl2);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  TimingScope ts("attn_bwd_dq", stream);
  hipLaunchKernelGGL((attn_bwd_dq_dma_kernel<DP, PADQ>), grid, dim3(256), 0, stream, k, (const float*)ds, dq, L, unp,
                     scale);
  return hipGetLastError();
}

template <int DP, bool VEC>
hipError_t bwd_fused_t(const float* q, const float* k, const float* v, const float* o,
                       const float* d_o, const float* lse, float* dq, float* dk, float* dv,
                       float* delta, float* ds, const View& L, float scale, hipStream_t stream) {
  constexpr int NWQ = 4, NWK = 4;
  const float sl2 = (float)((double)scale * 1.4426950408889634);
  const int n_qt = (L.T + NWQ * 16 - 1) / (NWQ * 16);
  const int n_kt = (L.T + NWK * 16 - 1) / (NWK * 16);
  hipError_t e;
  {
    TimingScope ts("attn_bwd_delta", stream);
    e = delta_launch(o, d_o, delta, L, stream);
  }
  if (e != hipSuccess) return e;
  if (ds != nullptr) {
    {
      TimingScope ts("attn_bwd_dkv", stream);
      hipLaunchKernelGGL((attn_bwd_dkv_kernel<DP, NWK, VEC, false, true>), dim3((unsigned)(n_kt * L.B * L.H)),
                         dim3(NWK * 64), 0, stream, q, k, v, d_o, lse, (const float*)delta,
                         (const float*)nullptr, dk, dv, ds, L, scale, sl2);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    TimingScope ts("attn_bwd_dq", stream);
    constexpr int NWD = WHA_DQ_NW;
    const int n_qt_d = (L.T + NWD * 16 - 1) / (NWD * 16);
    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<DP, NWD, VEC>), dim3((unsigned)(n_qt_d * L.B * L.H)),
                       dim3(NWD * 64), 0, stream, k, (const float*)ds, dq, L, scale);
    return hipGetLastError();
  }
  {
    TimingScope ts("attn_bwd_dq", stream);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<DP, NWQ, VEC, kFused>), dim3((unsigned)(n_qt * L.B * L.H)),
                       dim3(NWQ * 64), 0, stream, q, k, v, d_o, lse, delta, (const float*)nullptr, dq, L,
                       scale, sl2);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  {
    TimingScope ts("attn_bwd_dkv", stream);
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<DP, NWK, VEC, false, false>), dim3((unsigned)(n_kt * L.B * L.H)),
                       dim3(NWK * 64), 0, stream, q, k, v, d_o, lse, (const float*)delta,
                       (const float*)nullptr, dk, dv, (float*)nullptr, L, scale, sl2);
  }
  return hipGetLastError();
}

// (timed as attn_bwd_probs_*_rs: register-staged, told apart from the
// direct-to-LDS path below)
template <int DP, bool VEC, bool AV>
hipError_t bwd_probs_t(const float* d_o, const float* q, const float* k, const float* v,
                       const float* att, float* dq, float* dk, float* dv, float* delta, float* ds,
                       const View& L, float scale, hipStream_t stream) {
  constexpr int NWQ = 4, NWK = 4;
  const int n_qt = (L.T + NWQ * 16 - 1) / (NWQ * 16);
  const int n_kt = (L.T + NWK * 16 - 1) / (NWK * 16);
  {
    TimingScope ts("attn_bwd_probs_delta_rs", stream);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<DP, NWQ, VEC, kDeltaFromProbs, AV>),
                       dim3((unsigned)(n_qt * L.B * L.H)), dim3(NWQ * 64), 0, stream, q, k, v, d_o,
                       (const float*)nullptr, delta, att, (float*)nullptr, L, scale, 0.f);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (ds != nullptr) {
    // dK, dV and the dS tiles in one key-stationary pass; dQ = scale * dS K from them
    {
      TimingScope ts("attn_bwd_probs_dkv_rs", stream);
      hipLaunchKernelGGL((attn_bwd_dkv_kernel<DP, NWK, VEC, true, true>), dim3((unsigned)(n_kt * L.B * L.H)),
                         dim3(NWK * 64), 0, stream, q, k, v, d_o, (const float*)nullptr,
                         (const float*)delta, att, dk, dv, ds, L, scale, 0.f);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    TimingScope ts("attn_bwd_probs_dq_rs", stream);
    constexpr int NWD = WHA_DQ_NW;
    const int n_qt_d = (L.T + NWD * 16 - 1) / (NWD * 16);
    hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<DP, NWD, VEC>), dim3((unsigned)(n_qt_d * L.B * L.H)),
                       dim3(NWD * 64), 0, stream, k, (const float*)ds, dq, L, scale);
    return hipGetLastError();
  }
  {
    TimingScope ts("attn_bwd_probs_dq_rs", stream);
    hipLaunchKernelGGL((attn_bwd_dq_kernel<DP, NWQ, VEC, kProbs, AV>), dim3((unsigned)(n_qt * L.B * L.H)),
                       dim3(NWQ * 64), 0, stream, q, k, v, d_o, (const float*)nullptr, delta, att, dq, L,
                       scale, 0.f);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  {
    TimingScope ts("attn_bwd_probs_dkv_rs", stream);
    hipLaunchKernelGGL((attn_bwd_dkv_kernel<DP, NWK, VEC, true, false>), dim3((unsigned)(n_kt * L.B * L.H)),
                       dim3(NWK * 64), 0, stream, q, k, v, d_o, (const float*)nullptr,
                       (const float*)delta, att, dk, dv, (float*)nullptr, L, scale, 0.f);
  }
  return hipGetLastError();
}

}  // namespace

size_t bwd_ds_floats(const View& L) { return (size_t)L.B * L.H * (size_t)ds_rows(L.T) * 64; }

hipError_t launch_attn_bwd_delta(const float* o, const float* d_o, float* delta, const View& L, const char* name,
                                 hipStream_t stream) {
  TimingScope ts(name, stream);
  return delta_launch(o, d_o, delta, L, stream);
}

hipError_t launch_dq_from_ds(const float* k, const float* ds, float* dq, const View& L, float scale,
                             const char* name, hipStream_t stream) {
  // instantiated for the 32-wide wave-attention features (16-byte aligned rows)
  if (L.D != kWaveFeatures) return hipErrorInvalidValue;
  constexpr int NWD = WHA_DQ_NW;
  const int n_qt = (L.T + NWD * 16 - 1) / (NWD * 16);
  TimingScope ts(name, stream);
  hipLaunchKernelGGL((attn_bwd_dq_ds_kernel<kWaveFeatures, NWD, true>), dim3((unsigned)(n_qt * L.B * L.H)),
                     dim3(NWD * 64), 0, stream, k, ds, dq, L, scale);
  return hipGetLastError();
}

hipError_t launch_attn_bwd(const float* q, const float* k, const float* v, const float* o,
                           const float* d_o, const float* lse, float* dq, float* dk, float* dv,
                           float* delta, float* ds, const View& L, bool vec, float scale,
                           hipStream_t stream, const float* sc) {
  if (sc != nullptr && (ds == nullptr || !WHA_DKV_DMA || !scores_kept(L, vec))) return hipErrorInvalidValue;
  if (sc == nullptr && ds != nullptr && small_problem(L))
    return launch_attn_bwd_small(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
  if (WHA_DKV_DMA && ds != nullptr && vec && ds_head_fits(L) && (sc != nullptr ? kept_head_dim(L.D) : dma_head_dim(L.D))) {
    if (L.D == 48) return bwd_dma_t<48, false>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
    if (L.D < 48) return bwd_dma_t<48, true>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
    if (L.D == 64) return bwd_dma_t<64, false>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
    if (L.D < 64) return bwd_dma_t<64, true>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
    if (L.D == 128) return bwd_dma_t<128, false>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
    return bwd_dma_t<128, true>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream, sc);
  }
#define WHA_BWD(DP)                                                                                 \
  return vec ? bwd_fused_t<DP, true>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream) \
             : bwd_fused_t<DP, false>(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, L, scale, stream)
  switch (padded_dim(L.D)) {
    case 48: WHA_BWD(48);
    case 64: WHA_BWD(64);
    case 128: WHA_BWD(128);
    default: return hipErrorInvalidValue;
  }
#undef WHA_BWD
}

namespace {
// Head dims dma_head_dim() accepts, 128-bit operands, dS buffer present: the
// Delta pass (dP and sum_j att dP, on the forward's tiles) writing the stats
// blocks, the direct-to-LDS key-stationary kernel reading P from att (dK, dV,
// dS), then dQ from dS.
template <int DP, bool PADQ, bool AV>
hipError_t bwd_probs_dma_t(const float* d_o, const float* q, const float* k, const float* v, const float* att,
                           float* dq, float* dk, float* dv, float* delta, float* stats, float* ds, const View& L,
                           float scale, hipStream_t stream) {
  hipError_t e;
  {
    TimingScope ts("attn_bwd_probs_delta", stream);
    e = launch_probs_delta_dma(d_o, v, att, stats, L, AV, stream);
  }
  if (e != hipSuccess) return e;
  const int unp = dma_unpaired(L);
  const dim3 grid((unsigned)(dma_tiles(L, unp) * L.B * L.H));
  {
    TimingScope ts("attn_bwd_probs_dkv", stream);
    hipLaunchKernelGGL((attn_bwd_dkv_dma_kernel<DP, true, PADQ, true, true>), grid, dim3(256), 0, stream, q, k, v,
                       d_o, (const float*)stats, dk, dv, ds, att, L, unp, scale, 0.f);
    e = hipGetLastError();
  }
  if (e != hipSuccess) return e;
  TimingScope ts("attn_bwd_probs_dq", stream);
  hipLaunchKernelGGL((attn_bwd_dq_dma_kernel<DP, PADQ>), grid, dim3(256), 0, stream, k, (const float*)ds, dq, L,
                     unp, scale);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_attn_bwd_probs(const float* d_o, const float* q, const float* k, const float* v,
                                 const float* att, float* dq, float* dk, float* dv, float* delta, float* stats,
                                 float* ds, const View& L, bool vec, float scale, hipStream_t stream) {
  // 128-bit att loads need every row start 16-byte aligned (the non-VEC build
  // keeps scalar loads: it only serves unaligned operands)
  const bool av = vec && L.T % 4 == 0 && (reinterpret_cast<uintptr_t>(att) & 15) == 0;
  if (WHA_DKV_DMA && vec && ds != nullptr && stats != nullptr && ds_head_fits(L) && dma_head_dim(L.D)) {
#define WHA_BWDP_DMA(DP, PADQ)                                                                                \
  return av ? bwd_probs_dma_t<DP, PADQ, true>(d_o, q, k, v, att, dq, dk, dv, delta, stats, ds, L, scale, stream) \
            : bwd_probs_dma_t<DP, PADQ, false>(d_o, q, k, v, att, dq, dk, dv, delta, stats, ds, L, scale, stream)
    if (L.D == 48) WHA_BWDP_DMA(48, false);
    if (L.D < 48) WHA_BWDP_DMA(48, true);
    if (L.D == 64) WHA_BWDP_DMA(64, false);
    if (L.D < 64) WHA_BWDP_DMA(64, true);
    if (L.D == 128) WHA_BWDP_DMA(128, false);
    WHA_BWDP_DMA(128, true);
#undef WHA_BWDP_DMA
  }
#define WHA_BWDP(DP)                                                                                           \
  return !vec ? bwd_probs_t<DP, false, false>(d_o, q, k, v, att, dq, dk, dv, delta, ds, L, scale, stream)    \
         : av ? bwd_probs_t<DP, true, true>(d_o, q, k, v, att, dq, dk, dv, delta, ds, L, scale, stream)      \
              : bwd_probs_t<DP, true, false>(d_o, q, k, v, att, dq, dk, dv, delta, ds, L, scale, stream)
  switch (padded_dim(L.D)) {
    case 48: WHA_BWDP(48);
    case 64: WHA_BWDP(64);
    case 128: WHA_BWDP(128);
    default: return hipErrorInvalidValue;
  }
#undef WHA_BWDP
}

}  // namespace wha
