// Causal attention forward and backward for small problems (gfx950, fp32 MFMA).
//
// Same results as attn_fwd.hip / attn_bwd.hip (the core of attention_cpu,
// reference src/common/compute.rs:377-409, and attention_backward_single,
// src/cpu/backward.rs:313-363), for problems with few (b,h) heads and short
// rows: there the 64-row tile kernels launch fewer blocks than the chip has
// CUs (the 168-dim config: 16 heads x 4 tiles = 64 blocks for 256 CUs) and
// every block walks its causal sweep serially, so the step is latency-bound.
//
// Here a block covers 16 rows of one (b,h) with kSW waves (8; 4 at head dim
// 128), and the causal sweep of those rows is split over the waves: wave w
// takes the 16-row chunks w, w+kSW, ... of the other operand and keeps its own
// partial state; the partials merge through LDS in a fixed order
// (deterministic).  Grid = B*H*ceil(T/16) blocks per kernel, two kernels per
// step instead of four:
//   attn_fwd_small_kernel  O and LSE (online softmax per wave, LSE merge)
//   attn_bwd_small_kernel  dK, dV (key-stationary) and dQ (query-stationary,
//                          S and dP recomputed) of the block's 16 rows in one
//                          launch; Delta = dO.O formed in place (no
//                          statistics pass, no dS workspace)
// Each wave stages its chunk's operands in its own LDS region: a 16-row chunk
// is read from global memory row by row (consecutive lanes on consecutive
// units of 4, 2 or 1 head-dim entries, so every load instruction touches a
// few rows), and the next chunk's loads are in flight while the current chunk
// is consumed.
// From LDS each lane takes the two MFMA layouts the contractions need:
//   row fragment     lane (lq, g) holds row lq, d = g*DG .. g*DG+DG-1
//                    (A/B operands of contractions over the head dimension)
//   column fragment  lane (lq, g) holds rows 4g+i (i < 4), d = NDT*lq+dt
//                    (A operand of contractions over rows; the accumulators
//                    then hold d = NDT*(4g+i)+dt, the layout store_row_frag writes)
// Head dims pad to DP = 48, 64 or 128 with zeros; any stride (the unit width
// follows the strides and the tensors' alignment).
#include <algorithm>
#include <cstdint>
#include <initializer_list>
#include <type_traits>

#include "wha_launch.hpp"

namespace wha {

namespace {

// Waves per block: 8, or 4 at head dim 128 (the VGPR budget of its fragments).
template <int DP>
constexpr int kSWof = DP == 128 ? 4 : 8;

// A 16-row chunk is read as units of VEC consecutive head-dim entries (VEC =
// 4, 2 or 1, the widest the view's strides and alignment allow): unit
// lane + 64p, in row-major [16][DP / VEC] order, is row (lane + 64p) / E,
// entries VEC * ((lane + 64p) % E) .. +VEC-1, E = DP / VEC.  The (row, entry)
// pair of a lane repeats every PERIOD units, ROWS rows further on, so a lane
// needs PERIOD offsets, computed once: its loads add a uniform row step and
// its LDS stores an immediate.
template <int DP, int VEC>
struct ChunkLanes {
  static constexpr int E = DP / VEC;
  static constexpr int G = E % 64 == 0 ? 64 : E % 32 == 0 ? 32 : E % 16 == 0 ? 16 : E % 8 == 0 ? 8 : 4;  // gcd(E, 64)
  static constexpr int PERIOD = E / G;
  static constexpr int ROWS = 64 * PERIOD / E;
  static constexpr int PER = 16 * E / 64;  // units per lane
  static_assert(DP % VEC == 0 && PER % PERIOD == 0, "chunk unit layout");
  int goff[PERIOD];  // bytes from the chunk's first row; past D: kOutside
  int loff[PERIOD];  // floats into a [16][DP + 4] LDS tile
  // above every record count (rows of a head span < 2^31 bytes)
  static constexpr int kOutside = (int)0x80000000u;
  __device__ __forceinline__ ChunkLanes(int lane, int D, int st) {
#pragma unroll
    for (int j = 0; j < PERIOD; ++j) {
      const int idx = lane + 64 * j, row = idx / E, d = VEC * (idx % E);
      goff[j] = d < D ? 4 * (row * st + d) : kOutside;
      loff[j] = row * (DP + 4) + d;
    }
  }
};

// A 16-row chunk of one tensor in a wave's registers (unit p as above); zero
// past T and D.  Loads are raw buffer loads against a record that ends at
// the last valid entry of row T-1: an offset of a row at or past T is at least
// (T - row0) * st >= its end (st >= D), and units past D carry kOutside, so
// both read as zero (VEC divides D, so no unit straddles the end of a row).
// Requires T * st * 4 < 2^31 (checked by small_problem; also for 16 rows, so
// that no offset wraps) and row0 < T.
template <int DP, int VEC>
struct ChunkRaw {
  using Lanes = ChunkLanes<DP, VEC>;
  static constexpr int PER = Lanes::PER;
  float r[PER * VEC];
  __device__ __forceinline__ void load(const float* __restrict__ head, int row0, int T, int D, int st,
                                       const Lanes& cl) {
    typedef unsigned uintx2 __attribute__((ext_vector_type(2)));
    typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
    const int bytes = 4 * ((T - 1 - row0) * st + D);
    const __amdgpu_buffer_rsrc_t rs = buffer_rsrc(head + (int64_t)row0 * st, (uint32_t)bytes);
    const int step = 4 * Lanes::ROWS * st;
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int off = cl.goff[p % Lanes::PERIOD] + (p / Lanes::PERIOD) * step;
      if constexpr (VEC == 4) {
        const uintx4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
#pragma unroll
        for (int e = 0; e < 4; ++e) r[4 * p + e] = __uint_as_float(v[e]);
      } else if constexpr (VEC == 2) {
        const uintx2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
        r[2 * p] = __uint_as_float(v[0]);
        r[2 * p + 1] = __uint_as_float(v[1]);
      } else {
        r[p] = buffer_load_float(rs, off, 0);
      }
    }
  }
  // into a [16][DP + 4] LDS tile
  __device__ __forceinline__ void store(float* tile, const Lanes& cl) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      float* t = tile + cl.loff[p % Lanes::PERIOD] + (p / Lanes::PERIOD) * Lanes::ROWS * (DP + 4);
      if constexpr (VEC == 4) {
        *reinterpret_cast<float4*>(t) = make_float4(r[4 * p], r[4 * p + 1], r[4 * p + 2], r[4 * p + 3]);
      } else if constexpr (VEC == 2) {
        *reinterpret_cast<float2*>(t) = make_float2(r[2 * p], r[2 * p + 1]);
      } else {
        *t = r[p];
      }
    }
  }
};

// Orders a wave's LDS writes before its following LDS reads (and reads before
// later writes): the wave's lanes run in lockstep, so a wavefront-scope fence
// and a scheduling barrier suffice.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Row fragment of a [16][DP + 4] LDS tile: row lq, entries g*DG .. +DG-1, times mul.
template <int DP>
__device__ __forceinline__ void row_frag(const float* tile, int lq, int g, float mul, float* out) {
  constexpr int DG = DP / 4;
  const float* p = tile + lq * (DP + 4) + g * DG;
#pragma unroll
  for (int c = 0; c < DG / 4; ++c) {
    const float4 v = *reinterpret_cast<const float4*>(p + 4 * c);
    out[4 * c + 0] = v.x * mul;
    out[4 * c + 1] = v.y * mul;
    out[4 * c + 2] = v.z * mul;
    out[4 * c + 3] = v.w * mul;
  }
}

// Column fragment of a [16][DP + 4] LDS tile: rows 4g+i, entries NDT*lq + dt.
template <int DP>
__device__ __forceinline__ void col_frag(const float* tile, int lq, int g, float (&out)[4][DP / 16]) {
  constexpr int NDT = DP / 16;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) out[i][dt] = tile[(4 * g + i) * (DP + 4) + NDT * lq + dt];
  }
}

// Four consecutive entries (d .. d+3 of one row, d a multiple of 4) of a
// 16-row output to global memory: as two 8-byte stores when VEC >= 2 (D and
// the strides even, the tensor 8-byte aligned; VEC == 2 and D == d + 2 store
// the first pair only), else entry by entry below D.  No 16-byte store: its
// data registers need a wait state before they are overwritten, which this
// compiler does not always leave.
template <int VEC>
__device__ __forceinline__ void store_quad(float* __restrict__ p, int d, int D, float x0, float x1, float x2,
                                           float x3) {
  if constexpr (VEC >= 2) {
    if (d < D) *reinterpret_cast<float2*>(p) = make_float2(x0, x1);
    if (d + 2 < D) *reinterpret_cast<float2*>(p + 2) = make_float2(x2, x3);
  } else {
    if (d < D) p[0] = x0;
    if (d + 1 < D) p[1] = x1;
    if (d + 2 < D) p[2] = x2;
    if (d + 3 < D) p[3] = x3;
  }
}

// The waves' partial accumulators written to LDS by write_wave_part (wave w's
// tile at sm + w*TILE) are summed by the whole block, four consecutive output
// entries per thread, adding the waves in order (deterministic), and row r of
// the 16 goes to row row0 + r of dst, times mul.  Requires a __syncthreads()
// between the writes and this call.
template <int DP, int VEC>
__device__ __forceinline__ void store_wave_sums(const float* sm, float* __restrict__ dst, int row0, int T, int D,
                                                int64_t st, float mul) {
  constexpr int kSW = kSWof<DP>, TILE = 16 * (DP + 4);
  for (int e4 = threadIdx.x; e4 < 4 * DP; e4 += kSW * 64) {
    const int r = (4 * e4) / DP, d = (4 * e4) % DP;
    const int off = r * (DP + 4) + d;
    float4 x = *reinterpret_cast<const float4*>(sm + off);
#pragma unroll
    for (int w = 1; w < kSW; ++w) {
      const float4 y = *reinterpret_cast<const float4*>(sm + w * TILE + off);
      x.x += y.x;
      x.y += y.y;
      x.z += y.z;
      x.w += y.w;
    }
    if (row0 + r < T) store_quad<VEC>(dst + (int64_t)(row0 + r) * st + d, d, D, x.x * mul, x.y * mul, x.z * mul, x.w * mul);
  }
}

// A wave's accumulators acc[dt][i] = X[row lq][NDT*(4g+i)+dt] into its LDS tile.
template <int DP>
__device__ __forceinline__ void write_wave_part(float* tile, const floatx4 (&acc)[DP / 16], int lq, int g) {
  constexpr int NDT = DP / 16;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) tile[lq * (DP + 4) + NDT * (4 * g + i) + dt] = acc[dt][i];
  }
}

}  // namespace

template <int DP, int VEC>
__global__ __launch_bounds__(kSWof<DP> * 64) void attn_fwd_small_kernel(const float* __restrict__ Q,
                                                                       const float* __restrict__ K,
                                                                       const float* __restrict__ V,
                                                                       float* __restrict__ O,
                                                                       float* __restrict__ LSE, View L,
                                                                       float scale_log2) {
  constexpr int DG = DP / 4, NDT = DP / 16, kSW = kSWof<DP>, TILE = 16 * (DP + 4);
  // per wave: its K and V chunk tiles; after the sweep the first of them holds
  // the wave's partial output for the merge
  __shared__ __align__(16) float stage[kSW][2][TILE];
  __shared__ __align__(16) float qs[TILE];
  __shared__ float sm_m[kSW][16], sm_l[kSW][16];

  const int BH = L.B * L.H;
  const int n_g = (L.T + 15) / 16;
  const int bh = blockIdx.x % BH;
  const int qg = n_g - 1 - (int)(blockIdx.x / BH);  // the longest rows first
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int tid = threadIdx.x;
  // wave index as a scalar: conditions derived from it compile to scalar
  // branches, never to EXEC-masked blocks (which MFMAs would not respect)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int st = (int)L.st;  // < 2^29 (small_problem)
  const ChunkLanes<DP, VEC> cl(lane, L.D, st);
  const int qrow = 16 * qg + lq;            // this lane's query (MFMA column)
  const int key_last = min(qrow, L.T - 1);  // keys after it are masked
  float* ks = stage[wave][0];
  float* vs = stage[wave][1];

  // each wave's first K, V chunk, then the block's 16 queries, staged once by
  // wave 0 (its K and V loads in flight behind them)
  ChunkRaw<DP, VEC> kr, vr;
  if (wave <= qg) {
    kr.load(K + base, 16 * wave, L.T, L.D, st, cl);
    vr.load(V + base, 16 * wave, L.T, L.D, st, cl);
  }
  if (wave == 0) {
    ChunkRaw<DP, VEC> qr;
    qr.load(Q + base, 16 * qg, L.T, L.D, st, cl);
    qr.store(qs, cl);
  }
  __syncthreads();
  float qf[DG];
  row_frag<DP>(qs, lq, g, scale_log2, qf);

  // Running max m of this wave's chunks: started at its first chunk from an
  // anchor (the query's score against the chunk's first key) and moved only
  // by exact steps; every chunk's S accumulators start from -m, so the fused
  // multiply-add chain of the MFMA keeps its partial sums near 0 instead of
  // rounding scores of tens of units at every step.  A wave with no chunk
  // keeps m = -inf.
  float m = -INFINITY, l = 0.f;
  floatx4 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int c = wave; c <= qg; c += kSW) {
    kr.store(ks, cl);
    vr.store(vs, cl);
    wave_lds_sync();
    if (c == wave) {
      float kfa[DG];
      row_frag<DP>(ks, 0, g, 1.f, kfa);
      float a = 0.f;
#pragma unroll
      for (int j = 0; j < DG; ++j) a = fmaf(qf[j], kfa[j], a);
      m = pair_sum32(pair_sum16(a));  // identical in the query's four lane groups
    }
    {  // the next chunk's loads in flight during this one (clamped: every
       // trip issues the same loads, so no register copies merge paths)
      const int cn = min(c + kSW, qg);
      WHA_FENCE();
      kr.load(K + base, 16 * cn, L.T, L.D, st, cl);
      vr.load(V + base, 16 * cn, L.T, L.D, st, cl);
      WHA_FENCE();
    }
    const int key0 = 16 * c;  // <= 16*qg <= T-1: the chunk's first key is valid for every query here
    // S^T[key][query] - m (log2 units): lane element i = key key0+4g+i, query
    // qrow; the K fragment is read inside, so it is not held across the trips
    floatx4 s;
    auto scores = [&]() {
      float kf[DG];
      row_frag<DP>(ks, lq, g, 1.f, kf);
      s = floatx4{-m, -m, -m, -m};
#pragma unroll
      for (int j = 0; j < DG; ++j) s = mfma4(kf[j], qf[j], s);
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = (key0 + 4 * g + i > key_last) ? -INFINITY : s[i];
    };
    // The chunk's first key is valid for every query here, so mx is finite,
    // and >= 0 in the first chunk (the anchor's key).  Scores far above the
    // maximum they started from were summed at their own size: then the
    // chunk's scores are formed again from the new maximum (a second trip,
    // whose scores are all <= 0).
    float alpha = 1.f, dd;
    for (;;) {
      scores();
      float mx = -INFINITY;
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[i]);
      const bool redo = __builtin_amdgcn_ballot_w64(mx > kRedoMax) != 0;
      mx = pair_max32(pair_max16(mx));
      const float m_new = m + fmaxf(mx, 0.f);
      dd = m_new - m;  // exact step of the float maximum
      alpha *= fast_exp2(-dd);
      if (!redo) break;
      m = m_new;
    }
    const float m_new = m + dd;
    float vv[4][NDT];
    col_frag<DP>(vs, lq, g, vv);
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float p = fast_exp2(s[i] - dd);
      s[i] = p;
      rs += p;
    }
    l = l * alpha + rs;
    m = m_new;
    // O^T[d][query] += V^T[d][key] P^T[key][query], MFMA k-index g <-> key key0+4g+i
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma4(vv[i][dt], s[i], oacc[dt]);
    }
    wave_lds_sync();  // this chunk's tiles are read before the next one overwrites them
  }

  wait_vmem();  // the last trip's clamped prefetch lands before the wave can end
  // merge the waves' (max, sum, O) of each query: weights 2^(m_w - M);
  // a wave with no chunk keeps m = -inf and weighs zero
  const float lt = pair_sum32(pair_sum16(l));
  if (g == 0) {
    sm_m[wave][lq] = m;
    sm_l[wave][lq] = lt;
  }
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) ks[lq * (DP + 4) + NDT * (4 * g + i) + dt] = oacc[dt][i];
  }
  __syncthreads();
  // Four consecutive entries of one query row per thread: the row's wave
  // weights 2^(m_w - M) and 1 / sum (formed by every thread of the row, no
  // second barrier), then the weighted sum of the waves' partials in wave
  // order; the thread with the row's first entries writes its LSE.
  for (int e4 = tid; e4 < 4 * DP; e4 += kSW * 64) {
    const int r = (4 * e4) / DP, d = (4 * e4) % DP;
    const int off = r * (DP + 4) + d;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kSW; ++w) M = fmaxf(M, sm_m[w][r]);
    float wt[kSW], Ls = 0.f;
#pragma unroll
    for (int w = 0; w < kSW; ++w) {
      wt[w] = fast_exp2(sm_m[w][r] - M);
      Ls += wt[w] * sm_l[w][r];
    }
    const float inv = 1.f / Ls;
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < kSW; ++w) {
      const float4 y = *reinterpret_cast<const float4*>(&stage[w][0][off]);
      acc.x += wt[w] * y.x;
      acc.y += wt[w] * y.y;
      acc.z += wt[w] * y.z;
      acc.w += wt[w] * y.w;
    }
    const int q = 16 * qg + r;
    if (q < L.T) {
      if (d == 0 && LSE != nullptr) LSE[(int64_t)bh * L.T + q] = (M + log2f(Ls)) * kLn2;
      store_quad<VEC>(O + base + (int64_t)q * L.st + d, d, L.D, acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
    }
  }
}

// The backward in one launch.  Block kg owns keys 16kg .. 16kg+15 (dK, dV)
// and queries 16kg .. 16kg+15 (dQ); its tasks are
//   - query chunks kg .. n_g-1 of a key-stationary pass (lane column lq = key):
//     S = Q K^T and dP = dO V^T (contractions over d, queries on MFMA rows,
//     the accumulators started from -LSE/scale and -Delta), P =
//     exp2(S scale log2(e)), dS = P dP with Delta = dO.O of the chunk's rows
//     formed in place, then dV^T += dO^T P and dK^T += Q^T dS
//     (contractions over the chunk's rows); the diagonal chunk kg also gives
//     its queries' dQ^T += K^T dS^T from the same dS;
//   - key chunks 0 .. kg-1 of a query-stationary pass (lane column lq = query)
//     that forms S^T and dP^T the same way (P from the saved LSE, Delta of the
//     block's own queries) and dQ^T += K^T dS^T,
// n_g tasks for every block.  Task t goes to wave t % kSW, the
// key-stationary ones first; each wave keeps its partial dK, dV and dQ, and
// the partials merge through LDS in a fixed order (deterministic).  No dS
// leaves the chip.
template <int DP, int VEC>
__global__ __launch_bounds__(kSWof<DP> * 64) void attn_bwd_small_kernel(
    const float* __restrict__ Q, const float* __restrict__ K, const float* __restrict__ V,
    const float* __restrict__ O, const float* __restrict__ dO, const float* __restrict__ LSE, float* __restrict__ dQ,
    float* __restrict__ dK, float* __restrict__ dV, View L, float scale, float scale_log2) {
  constexpr int DG = DP / 4, NDT = DP / 16, kSW = kSWof<DP>, TILE = 16 * (DP + 4);
  // stage[s][w]: wave w's staged chunk s (Q, dO, O of a query chunk, or K, V of
  // a key chunk); after the sweep its partial dV (s = 0), dK (1), dQ (2).
  // own: the block's K, V rows (its keys) and Q, dO, O rows (its queries).
  __shared__ __align__(16) float stage[3][kSW][TILE];
  __shared__ __align__(16) float own[5][TILE];
  __shared__ __align__(16) float ds_t[16 * 20];  // the diagonal chunk's dS, transposed (pitch 20)

  const int BH = L.B * L.H;
  const int n_g = (L.T + 15) / 16;
  const int bh = blockIdx.x % BH;
  const int kg = (int)(blockIdx.x / BH);  // kg = 0 (the longest key-stationary sweep) first
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int tid = threadIdx.x;
  // wave index as a scalar: conditions derived from it compile to scalar
  // branches, never to EXEC-masked blocks (which MFMAs would not respect)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int st = (int)L.st;  // < 2^29 (small_problem)
  const ChunkLanes<DP, VEC> cl(lane, L.D, st);
  const int row = 16 * kg + lq;  // this lane's key (first pass) and query (second pass)
  const int n_kv = n_g - kg;     // key-stationary tasks
  // this wave's first query-stationary key chunk (>= kg: none)
  const int j0 = ((wave - n_kv) % kSW + kSW) % kSW;

  // the head's LSE row as a buffer: rows past T read as zero with no branch
  // (a branch around a load would make the compiler wait for every load in
  // flight, the prefetched chunk's included)
  const __amdgpu_buffer_rsrc_t lse_rs = buffer_rsrc(LSE + (int64_t)bh * L.T, (uint32_t)(4 * L.T));
  // Chunks in flight: Q, dO, O rows and raw LSE of the next key-stationary
  // task, K and V rows of the next query-stationary one.  The first of each
  // are requested before the block's own rows, so the three arrive together.
  ChunkRaw<DP, VEC> qr, dr, orr, kr, vr;
  float lsv[4];
  auto load_ks = [&](int c) {
    qr.load(Q + base, 16 * c, L.T, L.D, st, cl);
    dr.load(dO + base, 16 * c, L.T, L.D, st, cl);
    orr.load(O + base, 16 * c, L.T, L.D, st, cl);
#pragma unroll
    for (int i = 0; i < 4; ++i) lsv[i] = buffer_load_float(lse_rs, 4 * (16 * c + 4 * g + i), 0);
  };
  auto load_qs = [&](int c) {
    kr.load(K + base, 16 * c, L.T, L.D, st, cl);
    vr.load(V + base, 16 * c, L.T, L.D, st, cl);
  };
  if (wave < n_kv) load_ks(kg + wave);
  if (j0 < kg) load_qs(j0);
  const float lse_row = buffer_load_float(lse_rs, 4 * row, 0);  // the second pass's query

  for (int t = wave; t < 5; t += kSW) {
    const float* src = t == 0 ? K : t == 1 ? V : t == 2 ? Q : t == 3 ? dO : O;
    ChunkRaw<DP, VEC> r;
    r.load(src + base, 16 * kg, L.T, L.D, st, cl);
    r.store(own[t], cl);
  }
  __syncthreads();

  floatx4 dkacc[NDT], dvacc[NDT], dqacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
    dkacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
    dqacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  // ---- key-stationary tasks: query chunks c = kg + wave, kg + wave + kSW, ...
  if (wave < n_kv) {
    float* qs = stage[0][wave];
    float* os = stage[1][wave];  // dO
    float* ys = stage[2][wave];  // O
    // K unscaled: S is the plain dot product started from -LSE/scale, and
    // scale*log2(e) is applied per score in the exponent.  The forward's
    // rounding of q*scale*log2(e) is common to a row's keys; a per-key
    // rounding of K here would not be, and dQ = dS K amplifies such a
    // mismatch by the size of K.
    float kf[DG], vf[DG];
    row_frag<DP>(own[0], lq, g, 1.f, kf);
    row_frag<DP>(own[1], lq, g, 1.f, vf);
    const float inv_scale = 1.f / scale;
    for (int c = kg + wave; c < n_g; c += kSW) {
      const int q0 = 16 * c;
      qr.store(qs, cl);
      dr.store(os, cl);
      orr.store(ys, cl);
      float lse2[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) lse2[i] = -lsv[i] * inv_scale;
      wave_lds_sync();
      // the next chunk's loads in flight during this one (clamped: every trip
      // issues the same loads), kept ahead of the contractions by the fences
      WHA_FENCE();
      load_ks(min(c + kSW, n_g - 1));
      WHA_FENCE();

      float qf[DG], df[DG], qc[4][NDT], dc[4][NDT];
      row_frag<DP>(qs, lq, g, 1.f, qf);
      row_frag<DP>(os, lq, g, 1.f, df);
      col_frag<DP>(qs, lq, g, qc);
      col_frag<DP>(os, lq, g, dc);
      // Delta of query q0+lq (its d-range here, then the 4 lane groups); the
      // accumulator rows are queries q0+4g+i: their Delta from lanes 4g+i
      float dpart = 0.f;
      {
        float of[DG];
        row_frag<DP>(ys, lq, g, 1.f, of);
#pragma unroll
        for (int j = 0; j < DG; ++j) dpart += df[j] * of[j];
      }
      const float delta_lq = pair_sum32(pair_sum16(dpart));
      float dlt[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) dlt[i] = __shfl(delta_lq, 4 * g + i, 64);
      // S[query][key] - LSE/scale (dot-product units) and dP - Delta: lane
      // element i = query q0+4g+i, key row; started from the rows' -LSE/scale
      // and -Delta, so the large partial sums of S cancel in the first steps
      floatx4 s = floatx4{lse2[0], lse2[1], lse2[2], lse2[3]};
      floatx4 dp = floatx4{-dlt[0], -dlt[1], -dlt[2], -dlt[3]};
#pragma unroll
      for (int j = 0; j < DG; ++j) {
        s = mfma4(qf[j], kf[j], s);
        dp = mfma4(df[j], vf[j], dp);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = q0 + 4 * g + i;
        const bool valid = (q >= row) & (q < L.T) & (row < L.T);
        const float p = valid ? fast_exp2(s[i] * scale_log2) : 0.f;
        dp[i] = valid ? p * dp[i] : 0.f;
        s[i] = p;
      }
      // dV^T[d][key] += dO^T[d][query] P[query][key]; dK^T[d][key] += Q^T[d][query] dS[query][key]
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          dvacc[dt] = mfma4(dc[i][dt], s[i], dvacc[dt]);
          dkacc[dt] = mfma4(qc[i][dt], dp[i], dkacc[dt]);
        }
      }
      if (c == kg) {
        // The diagonal chunk (wave 0): its queries are the block's own, so
        // their dQ^T[d][query] += K^T[d][key] dS^T[key][query] comes from the
        // same dS, transposed through LDS: lane (lq, g) holds dS[query 4g+i]
        // [key lq]; the MFMA's k-index g <-> key 4g+i takes dS^T[key 4g+i]
        // [query lq].  No query-stationary task recomputes this chunk.
#pragma unroll
        for (int i = 0; i < 4; ++i) ds_t[(4 * g + i) * 20 + lq] = dp[i];
        wave_lds_sync();
        const float4 t4 = *reinterpret_cast<const float4*>(&ds_t[lq * 20 + 4 * g]);
        const float dst[4] = {t4.x, t4.y, t4.z, t4.w};
        float kc[4][NDT];
        col_frag<DP>(own[0], lq, g, kc);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = mfma4(kc[i][dt], dst[i], dqacc[dt]);
        }
      }
      wave_lds_sync();  // this chunk's tiles are read before the next one overwrites them
    }
  }

  // ---- query-stationary tasks: key chunk j is task n_kv + j, j = 0 .. kg-1
  if (j0 < kg) {
    float* ks = stage[0][wave];
    float* vs = stage[1][wave];
    float qf[DG], df[DG];
    row_frag<DP>(own[2], lq, g, scale_log2, qf);
    row_frag<DP>(own[3], lq, g, 1.f, df);
    float dpart = 0.f;  // Delta of query row
    {
      float of[DG];
      row_frag<DP>(own[4], lq, g, 1.f, of);
#pragma unroll
      for (int j = 0; j < DG; ++j) dpart += df[j] * of[j];
    }
    const float delta = pair_sum32(pair_sum16(dpart));
    const float lse2 = lse_row * kLog2e;
    for (int c = j0; c < kg; c += kSW) {
      const int key0 = 16 * c;
      kr.store(ks, cl);
      vr.store(vs, cl);
      wave_lds_sync();
      // the next chunk's loads in flight during this one (clamped)
      WHA_FENCE();
      load_qs(min(c + kSW, kg - 1));
      WHA_FENCE();
      float kf[DG], vf[DG], kc[4][NDT];
      row_frag<DP>(ks, lq, g, 1.f, kf);
      row_frag<DP>(vs, lq, g, 1.f, vf);
      col_frag<DP>(ks, lq, g, kc);
      // S^T[key][query] - LSE (log2 units) and dP^T - Delta: lane element i =
      // key key0+4g+i, query row; started from -LSE*log2(e) and -Delta (Q
      // carries the forward's scale*log2(e), as in the forward)
      floatx4 s = floatx4{-lse2, -lse2, -lse2, -lse2}, dp = floatx4{-delta, -delta, -delta, -delta};
#pragma unroll
      for (int j = 0; j < DG; ++j) {
        s = mfma4(kf[j], qf[j], s);
        dp = mfma4(vf[j], df[j], dp);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = (key0 + 4 * g + i <= row) & (row < L.T);
        const float p = valid ? fast_exp2(s[i]) : 0.f;
        dp[i] = valid ? p * dp[i] : 0.f;
      }
      // dQ^T[d][query] += K^T[d][key] dS^T[key][query], k-index g <-> key key0+4g+i
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) dqacc[dt] = mfma4(kc[i][dt], dp[i], dqacc[dt]);
      }
      wave_lds_sync();  // this chunk's tiles are read before the next one overwrites them
    }
  }

  wait_vmem();      // the last trips' clamped prefetches land before the wave can end
  __syncthreads();  // every wave is done with its staged chunks
  write_wave_part<DP>(stage[0][wave], dvacc, lq, g);
  write_wave_part<DP>(stage[1][wave], dkacc, lq, g);
  write_wave_part<DP>(stage[2][wave], dqacc, lq, g);
  __syncthreads();
  store_wave_sums<DP, VEC>(&stage[0][0][0], dV + base, 16 * kg, L.T, L.D, L.st, 1.f);
  store_wave_sums<DP, VEC>(&stage[1][0][0], dK + base, 16 * kg, L.T, L.D, L.st, scale);
  store_wave_sums<DP, VEC>(&stage[2][0][0], dQ + base, 16 * kg, L.T, L.D, L.st, scale);
}

bool small_problem(const View& L) {
  // the split-sweep kernels address a head's rows, and a chunk's 16, with
  // 32-bit byte offsets below 2^31
  return (int64_t)L.B * L.H * ((L.T + 63) / 64) < kSmallBlocks && L.T <= kSmallMaxT && padded_dim(L.D) != 0 &&
         (int64_t)std::max(L.T, 16) * L.st * 4 < ((int64_t)1 << 31);
}

namespace {
// The widest chunk unit (4, 2 or 1 floats) that the view's strides, the head
// dim and every tensor's alignment allow.
int small_vec(const View& L, std::initializer_list<const void*> ptrs) {
  for (int vec : {4, 2}) {
    bool ok = L.D % vec == 0 && L.st % vec == 0 && L.sh % vec == 0 && L.sb % vec == 0;
    for (const void* p : ptrs) ok = ok && reinterpret_cast<uintptr_t>(p) % (4 * vec) == 0;
    if (ok) return vec;
  }
  return 1;
}

template <int DP, int VEC>
hipError_t fwd_small_t(const float* q, const float* k, const float* v, float* o, float* lse, const View& L,
                       float scale, hipStream_t stream) {
  const float sl2 = (float)((double)scale * 1.4426950408889634);
  const dim3 grid((unsigned)((int64_t)L.B * L.H * ((L.T + 15) / 16)));
  TimingScope ts("attn_fwd", stream);
  hipLaunchKernelGGL((attn_fwd_small_kernel<DP, VEC>), grid, dim3(kSWof<DP> * 64), 0, stream, q, k, v, o, lse, L,
                     sl2);
  return hipGetLastError();
}

template <int DP, int VEC>
hipError_t bwd_small_t(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                       const float* lse, float* dq, float* dk, float* dv, const View& L, float scale,
                       hipStream_t stream) {
  const float sl2 = (float)((double)scale * 1.4426950408889634);
  const dim3 grid((unsigned)((int64_t)L.B * L.H * ((L.T + 15) / 16)));
  TimingScope ts("attn_bwd_dkv", stream);  // dK, dV and dQ
  hipLaunchKernelGGL((attn_bwd_small_kernel<DP, VEC>), grid, dim3(kSWof<DP> * 64), 0, stream, q, k, v, o, d_o, lse,
                     dq, dk, dv, L, scale, sl2);
  return hipGetLastError();
}

template <int DP>
hipError_t fwd_small_d(const float* q, const float* k, const float* v, float* o, float* lse, const View& L,
                       float scale, hipStream_t stream) {
  switch (small_vec(L, {q, k, v, o})) {
    case 4: return fwd_small_t<DP, 4>(q, k, v, o, lse, L, scale, stream);
    case 2: return fwd_small_t<DP, 2>(q, k, v, o, lse, L, scale, stream);
    default: return fwd_small_t<DP, 1>(q, k, v, o, lse, L, scale, stream);
  }
}

template <int DP>
hipError_t bwd_small_d(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                       const float* lse, float* dq, float* dk, float* dv, const View& L, float scale,
                       hipStream_t stream) {
  switch (small_vec(L, {q, k, v, o, d_o, dq, dk, dv})) {
    case 4: return bwd_small_t<DP, 4>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
    case 2: return bwd_small_t<DP, 2>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
    default: return bwd_small_t<DP, 1>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
  }
}
}  // namespace

hipError_t launch_attn_fwd_small(const float* q, const float* k, const float* v, float* o, float* lse,
                                 const View& L, float scale, hipStream_t stream) {
  switch (padded_dim(L.D)) {
    case 48: return fwd_small_d<48>(q, k, v, o, lse, L, scale, stream);
    case 64: return fwd_small_d<64>(q, k, v, o, lse, L, scale, stream);
    case 128: return fwd_small_d<128>(q, k, v, o, lse, L, scale, stream);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attn_bwd_small(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                                 const float* lse, float* dq, float* dk, float* dv, const View& L, float scale,
                                 hipStream_t stream) {
  switch (padded_dim(L.D)) {
    case 48: return bwd_small_d<48>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
    case 64: return bwd_small_d<64>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
    case 128: return bwd_small_d<128>(q, k, v, o, d_o, lse, dq, dk, dv, L, scale, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace wha
