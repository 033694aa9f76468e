// Wave (harmonic coherence) attention on gfx950: the attention the reference's
// training loop runs (src/common/attn.rs:72-430, called from
// src/cpu/forward.rs:113 and src/cpu/model_backward.rs:380-395).
//
// Per head h and positions q, k of one sequence the reference scores
//   score(q,k) = cos(n (phi_q - phi_k)) + cs * c_q . c_k       (attn.rs:200-207)
// with phi = atan2(s, r) of a 2-row projection of the input, c a C-row content
// projection, cs = 1/sqrt(C), n = softplus(harmonic_raw), over the mask
//   k <= q  and  (bucket(k) - bucket(q) mod 8 in {7, 0, 1}  or  k = q - 1)
// (attn.rs:167-224; bucket = phase_to_bucket, kv_cache.rs:66-70), then the
// causal softmax and the weighted sum of per-head value projections.
// Because cos(a - b) = cos a cos b + sin a sin b, the score is the dot product
// of per-position features f = [cos n phi, sin n phi, c] (with weight cs on the
// content part): a 32-wide (zero padded) MFMA contraction, after which the
// kernel family is the one of the dot-product path -- online softmax in the
// exp2 domain, 64-key LDS tiles, P V on MFMA -- with the bucket mask applied by
// a compare and select per score.
//
// Kernels
//   wave_feat_kernel      per position: phi, bucket, features   (1 thread / position)
//   wave_fwd_kernel       query-stationary fused forward: merged head outputs + LSE
//   wave_dkv_kernel       key-stationary backward: dV, dF_k (raw feature gradient
//                         of the key role) and dS to the workspace
//   (dF_q = dS F_k reuses the dot-product path's dQ-from-dS kernel with a 32-wide head)
//   wave_feat_bwd_kernel  per position: feature gradients -> d phi -> (d r, d s)
//                         through atan2, content gradients, harmonic partials
//   wave_harmonic_kernel  per head: deterministic sum of the harmonic partials
#include "wha_launch.hpp"

namespace wha {

namespace {
constexpr int kFP = kWaveFeatures;  // padded feature width
constexpr int kLDF = kFP + 4;       // LDS pitch of a feature tile

__device__ __forceinline__ float softplus_f(float x) { return x > 20.f ? x : logf(1.f + expf(x)); }
}  // namespace

// proj [B][T][H][P] (P = 2 + C: r, s, content) -> feat [B][H][T][32]
// (cos n phi, sin n phi, content, zeros), phase and bucket [B][H][T].
// Block = positions t0 .. t0+TT-1 of one b, all H heads.  Each position is
// computed by one thread in proj's order (consecutive threads read consecutive
// rows), staged in LDS head-major (odd pitch, conflict-free) and written out in
// the outputs' order: per head a contiguous run of TT feature rows, phases and
// buckets.
__global__ __launch_bounds__(256) void wave_feat_kernel(const float* __restrict__ proj,
                                                        const float* __restrict__ hraw, float* __restrict__ feat,
                                                        float* __restrict__ phase, int* __restrict__ bucket, int B,
                                                        int H, int T, int C, int C_used, int TT) {
  extern __shared__ float sm[];
  constexpr int FPITCH = kFP + 1;
  const int nbt = (T + TT - 1) / TT;
  const int b = (int)blockIdx.x / nbt, t0 = ((int)blockIdx.x % nbt) * TT;
  const int tn = min(TT, T - t0);
  const int P = 2 + C;
  const int npos = tn * H;
  float* fs = sm;                                // [H][tn][FPITCH]
  float* ps = sm + (size_t)H * TT * FPITCH;      // [H][tn] phase
  int* bs = reinterpret_cast<int*>(ps + H * TT);  // [H][tn] bucket
  const float* pblk = proj + ((int64_t)b * T + t0) * H * P;
  for (int pidx = threadIdx.x; pidx < npos; pidx += 256) {
    const int tt = pidx / H, h = pidx % H;
    const float* pr = pblk + (int64_t)pidx * P;
    const float phi = wave_phase(pr[1], pr[0]);
    const float n = softplus_f(hraw[h]);
    float sn, cn;
    sincosf(n * phi, &sn, &cn);
    float* f = fs + (h * tn + tt) * FPITCH;
    f[0] = cn;
    f[1] = sn;
    for (int j = 0; j < kFP - 2; ++j) {
      float v = 0.f;
      if (j < C_used) v = pr[2 + j];
      f[2 + j] = v;
    }
    ps[h * tn + tt] = phi;
    bs[h * tn + tt] = wave_phase_bucket(phi);
  }
  __syncthreads();
  // per head: tn feature rows (tn*8 float4), tn phases and buckets, each contiguous in memory
  for (int e = threadIdx.x; e < H * tn * (kFP / 4); e += 256) {
    const int r = e / (kFP / 4), q = e % (kFP / 4);  // r = h*tn + tt
    const int h = r / tn, tt = r % tn;
    const float* f = fs + r * FPITCH + 4 * q;
    const int64_t i = ((int64_t)b * H + h) * T + t0 + tt;
    reinterpret_cast<float4*>(feat + i * kFP)[q] = make_float4(f[0], f[1], f[2], f[3]);
  }
  for (int r = threadIdx.x; r < H * tn; r += 256) {
    const int h = r / tn, tt = r % tn;
    const int64_t i = ((int64_t)b * H + h) * T + t0 + tt;
    phase[i] = ps[r];
    bucket[i] = bs[r];
  }
}

// Fused forward.  Block = 16*NW queries of one (b,h), heaviest query tiles
// first; wave = 16 queries, one per lane, features pre-scaled by the score
// weights (1 for cos/sin, cs for content) and log2(e) as the MFMA B operand.
// Per 64-key tile: S^T = F_k F_q^T (keys on MFMA rows), bucket mask, online
// softmax, O^T += V^T P^T.  Every row attends to itself, so each output row has
// a positive softmax sum; the running max starts from a finite floor so that
// tiles whose scores are all masked leave the state unchanged.
template <int DP, int NW, bool VEC>
__global__ __launch_bounds__(NW * 64) void wave_fwd_kernel(const float* __restrict__ F,
                                                           const int* __restrict__ BK,
                                                           const float* __restrict__ V, float* __restrict__ O,
                                                           float* __restrict__ LSE, View Lv, float cs) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 16;
  constexpr int BN = 64;
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int NDT = DP / 16;
  constexpr int NKT = BN / 16;
  constexpr int FG = kFP / 4;
  __shared__ __align__(16) float Fs[BN * kLDF];
  __shared__ __align__(16) float Vs[BN * LD];
  __shared__ __align__(16) int Bs[BN];

  const int T = Lv.T;
  const int BH = Lv.B * Lv.H;
  const int n_qt = (T + BM - 1) / BM;
  const int bh = blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int q0 = qt * BM + wave * 16;
  const int qrow = q0 + lq;

  float qf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      qf[e] = qrow < T ? Fh[(int64_t)qrow * kFP + f] * (f < 2 ? kLog2e : w_cs) : 0.f;
    }
  }
  const int qb = qrow < T ? Bh[qrow] : 0;

  const int q_hi = min(T, (qt + 1) * BM);
  const int n_kt = (q_hi + BN - 1) / BN;

  TileStage<kFP, BN, NT, true> fs;
  TileStage<DP, BN, NT, VEC> vs;
  int kb_r = 0;
  fs.load(Fh, 0, T, kFP, kFP, tid);
  vs.load(V + vbase, 0, T, Lv.D, Lv.st, tid);
  if (tid < BN) kb_r = tid < T ? Bh[tid] : 0;

  float m_i = -1e30f, l_i = 0.f;
  floatx4 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < n_kt; ++kt) {
    __syncthreads();
    fs.template store<kLDF>(Fs, tid);
    vs.store_tile(Vs, tid);
    if (tid < BN) Bs[tid] = kb_r;
    __syncthreads();
    if (kt + 1 < n_kt) {
      const int nk = (kt + 1) * BN;
      fs.load(Fh, nk, T, kFP, kFP, tid);
      vs.load(V + vbase, nk, T, Lv.D, Lv.st, tid);
      if (tid < BN) kb_r = nk + tid < T ? Bh[nk + tid] : 0;
    }
    const int key0 = kt * BN;
    if (key0 > q0 + 15) continue;

    floatx4 s[NKT];
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) s[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < FG / 4; ++j) {
      float4 a[NKT];
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt)
        a[mt] = *reinterpret_cast<const float4*>(&Fs[(16 * mt + lq) * kLDF + g * FG + 4 * j]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].x, qf[4 * j + 0], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].y, qf[4 * j + 1], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].z, qf[4 * j + 2], s[mt]);
#pragma unroll
      for (int mt = 0; mt < NKT; ++mt) s[mt] = mfma4(a[mt].w, qf[4 * j + 3], s[mt]);
    }

    // mask: causal (key_lim), bucket relation or the previous position
    const int key_lim = min(qrow, T - 1) - key0;
    const int prev = qrow - 1 - key0;
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < NKT; ++mt) {
      const int4 kb4 = *reinterpret_cast<const int4*>(&Bs[16 * mt + 4 * g]);
      const int kbv[4] = {kb4.x, kb4.y, kb4.z, kb4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int kk = 16 * mt + 4 * g + i;
        const bool valid = (kk <= key_lim) & (wave_bucket_near(kbv[i], qb) | (kk == prev));
        const float x = valid ? s[mt][i] : -INFINITY;
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
  const float inv = qrow < T ? 1.f / l_sum : 0.f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] * inv;
  }
  store_row_frag<DP, VEC>(O + vbase, qrow, T, Lv.D, Lv.st, g, oacc, 1.f);
  if (LSE != nullptr && g == 0 && qrow < T) LSE[(int64_t)bh * T + qrow] = (m_i + log2f(l_sum)) * kLn2;
}

// Key-stationary backward: 64 keys of one (b,h) per block, 16 per wave (one
// per lane, features scaled as in the forward but on the key side, values as
// MFMA B operands).  Per 64-query tile: S and dP (queries on MFMA rows),
// P = exp2(S - LSE log2 e), dS = P (dP - Delta); dV^T += dO^T P and
// dF_k^T += F_q^T dS (raw, unweighted feature gradient; feature row m of d-tile
// dt is f = 2m + dt).  dS goes to the workspace in the dot-product path's layout.
template <int DP, bool VEC>
__global__ __launch_bounds__(256) void wave_dkv_kernel(const float* __restrict__ F, const int* __restrict__ BK,
                                                       const float* __restrict__ V, const float* __restrict__ dO,
                                                       const float* __restrict__ LSE,
                                                       const float* __restrict__ Delta, float* __restrict__ dF,
                                                       float* __restrict__ dV, float* __restrict__ DS, View Lv,
                                                       float cs) {
  constexpr int NT = 256;
  constexpr int BMQ = 64;
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int DG = DP / 4;
  constexpr int NDT = DP / 16;
  constexpr int NQT = BMQ / 16;
  constexpr int FG = kFP / 4;
  constexpr int NFT = kFP / 16;
  __shared__ __align__(16) float Fs[BMQ * kLDF];
  __shared__ __align__(16) float Os[BMQ * LD];
  __shared__ __align__(16) float lse_s[BMQ];
  __shared__ __align__(16) float del_s[BMQ];
  __shared__ __align__(16) int qb_s[BMQ];

  const int T = Lv.T;
  const int BH = Lv.B * Lv.H;
  const int bh = blockIdx.x % BH;
  const int kt = (int)(blockIdx.x / BH);
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;
  const int64_t rbase = (int64_t)bh * T;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int k0w = kt * 64 + wave * 16;
  const int krow = k0w + lq;

  float kf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      kf[e] = krow < T ? Fh[(int64_t)krow * kFP + f] * (f < 2 ? kLog2e : w_cs) : 0.f;
    }
  }
  float vf[DG];
  load_row_frag<DP, VEC>(V + vbase, krow, T, Lv.D, Lv.st, g, 1.f, vf);
  const int kb = krow < T ? Bh[krow] : 0;

  floatx4 dfacc[NFT], dvacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NFT; ++dt) dfacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int n_qt = (T + BMQ - 1) / BMQ;
  TileStage<kFP, BMQ, NT, true> fs;
  TileStage<DP, BMQ, NT, VEC> os;
  float lse_r = 0.f, del_r = 0.f;
  int qb_r = 0;
  auto load_tile = [&](int qt) {
    fs.load(Fh, qt * BMQ, T, kFP, kFP, tid);
    os.load(dO + vbase, qt * BMQ, T, Lv.D, Lv.st, tid);
    // raw LSE (scaled when stored to LDS): arithmetic on a value here would wait
    // for its load and, with it, for the tile loads issued just before
    if (tid < BMQ) {
      const int q = qt * BMQ + tid;
      lse_r = q < T ? LSE[rbase + q] : 0.f;
      del_r = q < T ? Delta[rbase + q] : 0.f;
      qb_r = q < T ? Bh[q] : 0;
    }
  };
  load_tile(kt);

  float* dsb = DS + ((int64_t)bh * ds_rows(T) + ds_block_row(kt, T) - (int64_t)64 * kt) * 64 + wave * 16 + lq;
  for (int qt = kt; qt < n_qt; ++qt) {
    __syncthreads();
    fs.template store<kLDF>(Fs, tid);
    os.store_tile(Os, tid);
    if (tid < BMQ) {
      lse_s[tid] = lse_r * kLog2e;
      del_s[tid] = del_r;
      qb_s[tid] = qb_r;
    }
    __syncthreads();
    if (qt + 1 < n_qt) load_tile(qt + 1);
    const int qbase = qt * BMQ;
    const int q_end = krow < T ? T : 0;  // valid queries: krow <= q < q_end

    floatx4 s[NQT], dp[NQT];
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
      s[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      dp[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int j = 0; j < FG / 4; ++j) {
      float4 a[NQT];
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt)
        a[mt] = *reinterpret_cast<const float4*>(&Fs[(16 * mt + lq) * kLDF + g * FG + 4 * j]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mt = 0; mt < NQT; ++mt) {
          const float av[4] = {a[mt].x, a[mt].y, a[mt].z, a[mt].w};
          s[mt] = mfma4(av[e], kf[4 * j + e], s[mt]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
      float4 c[NQT];
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt)
        c[mt] = lds_read_quad<DP>(Os, 16 * mt + lq, g * (DG / 4) + j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int mt = 0; mt < NQT; ++mt) {
          const float cv[4] = {c[mt].x, c[mt].y, c[mt].z, c[mt].w};
          dp[mt] = mfma4(cv[e], vf[4 * j + e], dp[mt]);
        }
      }
    }

    // lane element (mt,i): query qbase+16mt+4g+i, key krow
#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
      const float4 l4 = *reinterpret_cast<const float4*>(&lse_s[16 * mt + 4 * g]);
      const float4 d4 = *reinterpret_cast<const float4*>(&del_s[16 * mt + 4 * g]);
      const int4 b4 = *reinterpret_cast<const int4*>(&qb_s[16 * mt + 4 * g]);
      const float lq4[4] = {l4.x, l4.y, l4.z, l4.w};
      const float dq4[4] = {d4.x, d4.y, d4.z, d4.w};
      const int bq4[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = qbase + 16 * mt + 4 * g + i;
        const bool valid = (q >= krow) & (q < q_end) & (wave_bucket_near(kb, bq4[i]) | (q == krow + 1));
        float p = fast_exp2(s[mt][i] - lq4[i]);
        p = valid ? p : 0.f;
        s[mt][i] = p;
        dp[mt][i] = p * (dp[mt][i] - dq4[i]);
      }
    }

    {
      // rows up to T rounded up to 64 exist in the workspace: no per-row checks
      float* dsq = dsb + (int64_t)(qbase + 4 * g) * 64;
#pragma unroll
      for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
        for (int i = 0; i < 4; ++i) dsq[(16 * mt + i) * 64] = dp[mt][i];
      }
    }

#pragma unroll
    for (int mt = 0; mt < NQT; ++mt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float oa[NDT], fa[NFT];
        lds_read_seg<DP, NDT>(Os, 16 * mt + 4 * g + i, lq, oa);
        lds_read_vec<NFT>(&Fs[(16 * mt + 4 * g + i) * kLDF + NFT * lq], fa);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = mfma4(oa[dt], s[mt][i], dvacc[dt]);
#pragma unroll
        for (int dt = 0; dt < NFT; ++dt) dfacc[dt] = mfma4(fa[dt], dp[mt][i], dfacc[dt]);
      }
    }
  }

  store_row_frag<kFP, true>(dF + (int64_t)bh * T * kFP, krow, T, kFP, kFP, g, dfacc, 1.f);
  store_row_frag<DP, VEC>(dV + vbase, krow, T, Lv.D, Lv.st, g, dvacc, 1.f);
}

// Feature backward.  G = dF_q + dF_k (the score is symmetric in the two
// feature rows); dphi = n (cos nphi G1 - sin nphi G0); atan2's backward with the
// reference's guards (attn_backward.rs:203-218) gives d r, d s; the content
// gradient is cs G[2..]; the harmonic partial is phi * dphi / n.  Block =
// positions t0 .. t0+TT-1 of one b, all H heads: the head-major inputs (G rows,
// cos/sin, phase) are read as contiguous per-head runs and staged in LDS in
// proj's order (odd pitch), one thread per position computes its dproj row
// into LDS, the block's dproj rows (contiguous in memory) are written out
// coalesced, and the block's harmonic partial per head (its positions summed
// in order) goes to hpart[block][h].
__global__ __launch_bounds__(256) void wave_feat_bwd_kernel(const float* __restrict__ proj,
                                                            const float* __restrict__ feat,
                                                            const float* __restrict__ phase,
                                                            const float* __restrict__ dFq,
                                                            const float* __restrict__ dFk,
                                                            const float* __restrict__ hraw,
                                                            float* __restrict__ dproj, float* __restrict__ hpart,
                                                            int B, int H, int T, int C, float cs, int TT) {
  extern __shared__ float sm[];
  const int nbt = (T + TT - 1) / TT;
  const int b = (int)blockIdx.x / nbt, t0 = ((int)blockIdx.x % nbt) * TT;
  const int tn = min(TT, T - t0);
  const int P = 2 + C;
  const int P4 = (P + 3) / 4;                  // float4 pieces of a gradient row that hold G
  const int GP = (P + 3) | 1;                  // odd pitch: G[0..P-1], cos, sin, phi
  const int npos = tn * H;
  float* gs = sm;                              // [tn*H][GP], proj order
  float* ds = sm + (size_t)TT * H * GP;        // [tn*H][P]
  float* hs = ds + (size_t)TT * H * P;         // [tn*H] harmonic partials
  // G rows: per head, tn consecutive rows of 32 floats, the first 4*P4 used
  for (int e = threadIdx.x; e < H * tn * P4; e += 256) {
    const int r = e / P4, q = e % P4;          // r = h*tn + tt
    const int h = r / tn, tt = r % tn;
    const int64_t i = ((int64_t)b * H + h) * T + t0 + tt;
    const float4 x = reinterpret_cast<const float4*>(dFq + i * kFP)[q];
    const float4 y = reinterpret_cast<const float4*>(dFk + i * kFP)[q];
    float* g = gs + (tt * H + h) * GP + 4 * q;
    const float v[4] = {x.x + y.x, x.y + y.y, x.z + y.z, x.w + y.w};
#pragma unroll
    for (int k = 0; k < 4; ++k)
      if (4 * q + k < P) g[k] = v[k];
  }
  for (int r = threadIdx.x; r < H * tn; r += 256) {
    const int h = r / tn, tt = r % tn;
    const int64_t i = ((int64_t)b * H + h) * T + t0 + tt;
    const float2 cs2 = *reinterpret_cast<const float2*>(feat + i * kFP);
    float* g = gs + (tt * H + h) * GP + P;
    g[0] = cs2.x;
    g[1] = cs2.y;
    g[2] = phase[i];
  }
  __syncthreads();
  const float* pblk = proj + ((int64_t)b * T + t0) * H * P;
  for (int pidx = threadIdx.x; pidx < npos; pidx += 256) {
    const int h = pidx % H;
    const float* g = gs + pidx * GP;
    const float cn = g[P], sn = g[P + 1], phi = g[P + 2];
    const float u = cn * g[1] - sn * g[0];
    const float dphi = softplus_f(hraw[h]) * u;
    const float r0 = pblk[(int64_t)pidx * P], s0 = pblk[(int64_t)pidx * P + 1];
    const float mag_sq = r0 * r0 + s0 * s0;
    float d_r = 0.f, d_s = 0.f;
    if (fabsf(dphi) >= 1e-12f && mag_sq >= 1e-8f) {
      const float m = fmaxf(mag_sq, 1e-12f);
      d_r = dphi * (-s0 / m);
      d_s = dphi * (r0 / m);
    }
    float* d = ds + pidx * P;
    d[0] = d_r;
    d[1] = d_s;
    for (int j = 0; j < C; ++j) d[2 + j] = cs * g[2 + j];
    hs[pidx] = phi * u;
  }
  __syncthreads();
  float* dblk = dproj + ((int64_t)b * T + t0) * H * P;
  for (int e = threadIdx.x; e < npos * P; e += 256) dblk[e] = ds[e];
  if ((int)threadIdx.x < H) {
    float acc = 0.f;
    for (int tt = 0; tt < tn; ++tt) acc += hs[tt * H + threadIdx.x];
    hpart[(int64_t)blockIdx.x * H + threadIdx.x] = acc;
  }
}

// d_harmonic_raw[h] (+)= sigmoid(raw) * sum over the feature-backward blocks of
// hpart[block][h]: one block per head, fixed per-thread strides and a fixed
// tree, so the sum is deterministic (attn.rs:372, :418).
__global__ __launch_bounds__(256) void wave_harmonic_kernel(const float* __restrict__ hpart,
                                                            const float* __restrict__ hraw,
                                                            float* __restrict__ d_hraw, int nblk, int H) {
  __shared__ float red[256];
  const int h = blockIdx.x;
  float acc = 0.f;
  for (int j = threadIdx.x; j < nblk; j += 256) acc += hpart[(int64_t)j * H + h];
  red[threadIdx.x] = acc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) red[threadIdx.x] += red[threadIdx.x + w];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const float raw = hraw[h];
    d_hraw[h] = red[0] * (1.f / (1.f + expf(-raw)));
  }
}

// Rows of att_weights_all on demand (attn.rs:240): one block per (b*h, row)
// (b*h on grid.x, rows on grid.y),
// the query's features in LDS, one key per thread per pass;
// p = exp(score - lse) where the mask admits the key, 0 where it excludes a
// key j <= t, -inf after the diagonal (the reference's untouched entries).
__global__ __launch_bounds__(256) void wave_probs_rows_kernel(const float* __restrict__ F,
                                                              const int* __restrict__ BK,
                                                              const float* __restrict__ LSE, RowList rl,
                                                              float* __restrict__ out, int T, float cs) {
  __shared__ float qs[kFP];
  const int64_t bh = blockIdx.x;
  const int r = blockIdx.y;
  const int t = rl.rows[r];  // validated on the host: 0 <= t < T
  const float* Fh = F + bh * T * kFP;
  const int* Bh = BK + bh * T;
  if (threadIdx.x < kFP) qs[threadIdx.x] = Fh[(int64_t)t * kFP + threadIdx.x] * (threadIdx.x < 2 ? 1.f : cs);
  __syncthreads();
  const int qb = Bh[t];
  const float lse = LSE[bh * T + t];
  float* dst = out + (bh * rl.n + r) * T;
  for (int j = threadIdx.x; j < T; j += blockDim.x) {
    float p = -INFINITY;
    if (j <= t) {
      p = 0.f;
      if (wave_bucket_near(Bh[j], qb) || j == t - 1) {
        const float* kr = Fh + (int64_t)j * kFP;
        float dot = 0.f;
        for (int f = 0; f < kFP; ++f) dot += qs[f] * kr[f];
        p = expf(dot - lse);
      }
    }
    dst[j] = p;
  }
}

// ------------------------------------------------------------------ launchers

namespace {
// Positions per block of the feature kernels: the largest power of two up to 64
// whose LDS staging fits in kFeatLds bytes.
constexpr size_t kFeatLds = 40 * 1024;
size_t feat_fwd_lds(int H, int TT) { return (size_t)H * TT * (kFP + 1 + 2) * sizeof(float); }
size_t feat_bwd_lds(int H, int TT, int C) {
  const int P = 2 + C;
  return (size_t)H * TT * (((P + 3) | 1) + P + 1) * sizeof(float);
}
int feat_tile(int H, int T, size_t (*lds)(int, int, int), int C) {
  int tt = 64;
  while (tt > 1 && (lds(H, tt, C) > kFeatLds || tt >= 2 * T)) tt /= 2;
  return tt;
}
size_t feat_fwd_lds3(int H, int TT, int) { return feat_fwd_lds(H, TT); }
}  // namespace

hipError_t launch_wave_features(const float* proj, const float* hraw, float* feat, float* phase, int* bucket,
                                int B, int H, int T, int C, int C_used, hipStream_t stream) {
  const int tt = feat_tile(H, T, feat_fwd_lds3, C);
  if (feat_fwd_lds(H, tt) > kFeatLds) return hipErrorInvalidValue;  // more heads than one block stages
  const int nblk = B * ((T + tt - 1) / tt);
  TimingScope ts("wave_feat", stream);
  hipLaunchKernelGGL(wave_feat_kernel, dim3((unsigned)nblk), dim3(256), feat_fwd_lds(H, tt), stream, proj, hraw,
                     feat, phase, bucket, B, H, T, C, C_used, tt);
  return hipGetLastError();
}

template <int DP, bool VEC>
static hipError_t wave_fwd_t(const float* feat, const int* bucket, const float* v, float* merged, float* lse,
                             const View& Lv, float cs, hipStream_t stream) {
  constexpr int NW = 4;
  const int n_qt = (Lv.T + NW * 16 - 1) / (NW * 16);
  TimingScope ts("wave_fwd", stream);
  hipLaunchKernelGGL((wave_fwd_kernel<DP, NW, VEC>), dim3((unsigned)(n_qt * Lv.B * Lv.H)), dim3(NW * 64), 0,
                     stream, feat, bucket, v, merged, lse, Lv, cs);
  return hipGetLastError();
}

hipError_t launch_wave_fwd(const float* feat, const int* bucket, const float* v, float* merged, float* lse,
                           const View& Lv, bool vec, float cs, hipStream_t stream) {
  switch (padded_dim(Lv.D)) {
    case 48:
      return vec ? wave_fwd_t<48, true>(feat, bucket, v, merged, lse, Lv, cs, stream)
                 : wave_fwd_t<48, false>(feat, bucket, v, merged, lse, Lv, cs, stream);
    case 64:
      return vec ? wave_fwd_t<64, true>(feat, bucket, v, merged, lse, Lv, cs, stream)
                 : wave_fwd_t<64, false>(feat, bucket, v, merged, lse, Lv, cs, stream);
    case 128:
      return vec ? wave_fwd_t<128, true>(feat, bucket, v, merged, lse, Lv, cs, stream)
                 : wave_fwd_t<128, false>(feat, bucket, v, merged, lse, Lv, cs, stream);
    default:
      return hipErrorInvalidValue;
  }
}

template <int DP, bool VEC>
static hipError_t wave_dkv_t(const float* feat, const int* bucket, const float* v, const float* d_merged,
                             const float* lse, const float* delta, float* dfk, float* dv, float* ds, const View& Lv,
                             float cs, hipStream_t stream) {
  const int n_kt = (Lv.T + 63) / 64;
  TimingScope ts("wave_bwd_dkv", stream);
  hipLaunchKernelGGL((wave_dkv_kernel<DP, VEC>), dim3((unsigned)(n_kt * Lv.B * Lv.H)), dim3(256), 0, stream, feat,
                     bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs);
  return hipGetLastError();
}

hipError_t launch_wave_bwd_core(const float* feat, const int* bucket, const float* v, const float* merged,
                                const float* d_merged, const float* lse, float* delta, float* dfk, float* dfq,
                                float* dv, float* ds, const View& Lv, bool vec, float cs, hipStream_t stream) {
  hipError_t e = launch_attn_bwd_delta(merged, d_merged, delta, Lv, "wave_bwd_delta", stream);
  if (e != hipSuccess) return e;
  switch (padded_dim(Lv.D)) {
    case 48:
      e = vec ? wave_dkv_t<48, true>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : wave_dkv_t<48, false>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    case 64:
      e = vec ? wave_dkv_t<64, true>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : wave_dkv_t<64, false>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    case 128:
      e = vec ? wave_dkv_t<128, true>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : wave_dkv_t<128, false>(feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    default:
      return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  const int64_t F = kFP;
  const View Lf{Lv.B, Lv.H, Lv.T, kFP, (int64_t)Lv.H * Lv.T * F, (int64_t)Lv.T * F, F};
  return launch_dq_from_ds(feat, ds, dfq, Lf, 1.f, "wave_bwd_dq", stream);
}

hipError_t launch_wave_feat_bwd(const float* proj, const float* feat, const float* phase, const float* dfq,
                                const float* dfk, const float* hraw, float* dproj, float* hpart, float* d_hraw,
                                int B, int H, int T, int C, float cs, hipStream_t stream) {
  const int tt = feat_tile(H, T, feat_bwd_lds, C);
  if (feat_bwd_lds(H, tt, C) > kFeatLds) return hipErrorInvalidValue;  // more heads than one block stages
  const int nblk = B * ((T + tt - 1) / tt);
  {
    TimingScope ts("wave_feat_bwd", stream);
    hipLaunchKernelGGL(wave_feat_bwd_kernel, dim3((unsigned)nblk), dim3(256), feat_bwd_lds(H, tt, C), stream, proj,
                       feat, phase, dfq, dfk, hraw, dproj, hpart, B, H, T, C, cs, tt);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (d_hraw == nullptr) return hipSuccess;
  TimingScope ts("wave_harmonic", stream);
  hipLaunchKernelGGL(wave_harmonic_kernel, dim3((unsigned)H), dim3(256), 0, stream, (const float*)hpart, hraw,
                     d_hraw, nblk, H);
  return hipGetLastError();
}

hipError_t launch_wave_probs_rows(const float* feat, const int* bucket, const float* lse, const RowList& rl,
                                  float* out, int B, int H, int T, float cs, hipStream_t stream) {
  TimingScope ts("wave_probs_rows", stream);
  hipLaunchKernelGGL(wave_probs_rows_kernel, dim3((unsigned)(B * H), (unsigned)rl.n), dim3(256), 0, stream, feat,
                     bucket, lse, rl, out, T, cs);
  return hipGetLastError();
}

}  // namespace wha
