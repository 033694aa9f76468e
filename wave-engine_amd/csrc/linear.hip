// fp32 MFMA GEMM for the c_attn / c_proj projections around the attention core
// (gfx950), forward and backward.
//
// Reference semantics (one position at a time, sequential f32 sums):
//   linear / linear_batch      y[i] = b[i] + sum_j w[i][j] x[j]     src/common/compute.rs:441-453, model.rs:144-151
//   linear_backward_dx         d_x[j] = sum_i d_y[i] w[i][j]        src/common/math/backward.rs:36-46
//   outer_product_accum        d_w[i][j] = sum_pos d_y[pos][i] x[pos][j],  d_b[i] = sum_pos d_y[pos][i]
//                                                                   src/common/compute.rs:263-282
// Here all positions of a batch form one GEMM C[m][n] = bias[n] + sum_k A(m,k) B(k,n)
// with A and B given by strides, so the same kernel serves y = X W^T + b,
// dX = dY W and dW = dY^T X.
//
// Tiling: 128 x 128 (or 64 x 128, 64 x 64) output tile per 256-thread block,
// 2 x 2 waves; 32-deep k stages fetched straight into LDS by buffer loads
// (gemm_dma_kernel), or, where alignment or size rule those out, 16-deep stages
// staged through registers with the next stage prefetched (gemm_kernel).
// MFMA rows are output columns n and MFMA columns are output rows m,
// so each lane ends with 4 consecutive n of one row: 128-bit stores, bias added
// as a float4.  Lane group g covers k = 4g..4g+3 of a stage, so one 128-bit LDS
// read supplies four MFMA steps.  Split-K writes per-split partial tiles that a
// second kernel sums in a fixed order (deterministic).
#include "wha_launch.hpp"

// k depth of one LDS stage: 16 measured ahead of 32 (layer step 1.498 vs 1.505 ms,
// wave step 0.879 vs 0.888 ms) and 64 (1.525, 0.900 ms)
#ifndef WHA_GEMM_KT
#define WHA_GEMM_KT 16
#endif
// Direct-to-LDS stages (gemm_dma_kernel) where the operands allow them, and their k depth.
#ifndef WHA_GEMM_DMA
#define WHA_GEMM_DMA 1
#endif
#ifndef WHA_GEMM_DMA_KT
#define WHA_GEMM_DMA_KT 32
#endif
// 64 x 64 per-head projections on head64_gemm_kernel
#ifndef WHA_HEAD64
#define WHA_HEAD64 1
#endif

namespace wha {

namespace {
// Output columns per block: 64 per wave along n, WN = 2 waves along n (128
// columns) or WN = 1 (64 columns, for N <= 64: the per-head value projections).
constexpr int kGBN = 128;
}

struct GemmArgs {
  const float* a;
  int64_t a_sm, a_sk;  // A(m,k) = a[m*a_sm + k*a_sk]
  const float* b;
  int64_t b_sn, b_sk;  // B(k,n) = b[n*b_sn + k*b_sk]
  float* c;
  int64_t ldc;         // C(m,n) = c[m*ldc + n]  (or the split-K partial [z][M][N])
  const float* bias;   // [N] or nullptr
  int M, N, K;
  int k_chunk;         // k range per split (multiple of the stage depth)
  bool c_vec;          // c, ldc and c_sb allow 128-bit stores
  bool accumulate;     // C += result instead of C = result
  int batch = 1;       // independent GEMMs, operands offset by the strides below
  int splits = 1;      // blockIdx.z = batch index * splits + split index
  int64_t a_sb = 0, b_sb = 0, c_sb = 0, bias_sb = 0;
  bool a_vec = false;  // A's base, batch stride and row stride along its contiguous
  bool b_vec = false;  // direction are 16-byte multiples (set by gemm_t); same for B
  // Row sums of A over the k range (A k-contiguous only, i.e. the weight-gradient
  // GEMM, where they are the bias gradient): rowsum[bt*rowsum_sb + m] = sum_k A(m,k),
  // written by the blocks of the first column tile; with split-K each split writes
  // rowsum_part[(bt*splits + split)*M + m] and the reduce adds the splits in order.
  float* rowsum = nullptr;
  int64_t rowsum_sb = 0;
  float* rowsum_part = nullptr;
  // gemm_dma_kernel: bytes of one batch's A and B that its loads may touch
  // (the buffer descriptors' extents; set by gemm_dma_ok)
  uint32_t a_bytes = 0, b_bytes = 0;
};


// Staging of one ROWS x KT operand tile; element (r, k) of the source is
// p[r*s_r + k*s_k].  KC (s_k == 1, rows of the tile are source rows): LDS
// [ROWS][KT + 4], k contiguous.  Otherwise (s_r == 1, columns of the tile are
// source rows): LDS [KT][ROWS + 4], rows contiguous.  Either way each thread
// moves 128-bit pieces along the source's contiguous direction, so global loads
// are coalesced and LDS stores are 128-bit and conflict-free.
template <int ROWS, int KT, bool KC>
struct GemmStage {
  static constexpr int LDK = KT + 4;
  static constexpr int LDR = ROWS + 4;
  static constexpr int ELEMS = KC ? ROWS * LDK : KT * LDR;
  static constexpr int NF4 = ROWS * KT / 4;
  static constexpr int PER = NF4 / 256;
  static_assert(NF4 % 256 == 0, "tile must split evenly over 256 threads");
  float4 v[PER];
  // FULL: the whole ROWS x KT tile is in bounds and every piece 16-byte aligned
  // (decided per block), so each piece is one unpredicated 128-bit load.
  template <bool FULL>
  __device__ __forceinline__ void load(const float* p, int64_t s_r, int64_t s_k, int r0, int R,
                                       int k0, int k_end, int tid) {
    if constexpr (FULL) {
#pragma unroll
      for (int q = 0; q < PER; ++q) {
        const int idx = tid + 256 * q;
        if (KC) {
          const int rr = idx / (KT / 4), c = (idx % (KT / 4)) * 4;
          v[q] = *reinterpret_cast<const float4*>(p + (int64_t)(r0 + rr) * s_r + (k0 + c));
        } else {
          const int kr = idx / (ROWS / 4), rc = (idx % (ROWS / 4)) * 4;
          v[q] = *reinterpret_cast<const float4*>(p + (int64_t)(k0 + kr) * s_k + (r0 + rc));
        }
      }
      return;
    }
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = tid + 256 * q;
      float4 val = make_float4(0.f, 0.f, 0.f, 0.f);
      if (KC) {
        const int rr = idx / (KT / 4), c = (idx % (KT / 4)) * 4;
        const int r = r0 + rr, k = k0 + c;
        if (r < R) {
          const float* src = p + (int64_t)r * s_r + (int64_t)k * s_k;
          if (k + 3 < k_end && (((uintptr_t)src) & 15) == 0) {
            val = *reinterpret_cast<const float4*>(src);
          } else {
            if (k + 0 < k_end) val.x = src[0];
            if (k + 1 < k_end) val.y = src[1];
            if (k + 2 < k_end) val.z = src[2];
            if (k + 3 < k_end) val.w = src[3];
          }
        }
      } else {
        const int kr = idx / (ROWS / 4), rc = (idx % (ROWS / 4)) * 4;
        const int r = r0 + rc, k = k0 + kr;
        if (k < k_end) {
          const float* src = p + (int64_t)k * s_k + (int64_t)r * s_r;
          if (r + 3 < R && (((uintptr_t)src) & 15) == 0) {
            val = *reinterpret_cast<const float4*>(src);
          } else {
            if (r + 0 < R) val.x = src[0];
            if (r + 1 < R) val.y = src[1];
            if (r + 2 < R) val.z = src[2];
            if (r + 3 < R) val.w = src[3];
          }
        }
      }
      v[q] = val;
    }
  }
  // Sum of this thread's pieces (not KC: all of a thread's pieces cover the same
  // four rows rc..rc+3, rc = (tid % (ROWS/4))*4, at different k).
  __device__ __forceinline__ void add_to(float4& rs) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      rs.x += v[q].x;
      rs.y += v[q].y;
      rs.z += v[q].z;
      rs.w += v[q].w;
    }
  }
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int q = 0; q < PER; ++q) {
      const int idx = tid + 256 * q;
      if (KC) {
        const int rr = idx / (KT / 4), c = (idx % (KT / 4)) * 4;
        *reinterpret_cast<float4*>(lds + rr * LDK + c) = v[q];
      } else {
        const int kr = idx / (ROWS / 4), rc = (idx % (ROWS / 4)) * 4;
        *reinterpret_cast<float4*>(lds + kr * LDR + rc) = v[q];
      }
    }
  }
  // MFMA operand values of the TPW 16-row tiles a wave owns (rows rowbase ..
  // rowbase + 16*TPW) for k = ks + 4g + e, e = 0..3: out[t][e].  KC: tile t,
  // lane lq is row rowbase + 16t + lq (one 128-bit read per tile).  Otherwise
  // tile t, lane lq is row rowbase + TPW*lq + t (one TPW-wide read per e): the
  // row permutation the epilogue undoes.
  template <int TPW>
  __device__ __forceinline__ static void fetch(const float* lds, int rowbase, int ks, int lq, int g,
                                               float (&out)[TPW][4]) {
    if (KC) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const float4 x = *reinterpret_cast<const float4*>(&lds[(rowbase + 16 * t + lq) * LDK + ks + 4 * g]);
        out[t][0] = x.x;
        out[t][1] = x.y;
        out[t][2] = x.z;
        out[t][3] = x.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* src = &lds[(ks + 4 * g + e) * LDR + rowbase + TPW * lq];
        if (TPW == 4) {
          const float4 x = *reinterpret_cast<const float4*>(src);
          out[0][e] = x.x;
          out[1 % TPW][e] = x.y;
          out[2 % TPW][e] = x.z;
          out[3 % TPW][e] = x.w;
        } else {
#pragma unroll
          for (int t = 0; t < TPW; ++t) out[t][e] = src[t];
        }
      }
    }
  }
  // Row (within the wave's rows) of tile t, MFMA row/column index j.
  __device__ __forceinline__ static int row_of(int t, int j, int tpw) { return KC ? 16 * t + j : tpw * j + t; }
};

// MFMA work of one KT-deep stage held in LDS.
template <int BM, int KT, int WN, bool A_KC, bool B_KC>
__device__ __forceinline__ void gemm_stage_mfma(const float* As, const float* Bs,
                                                floatx4 (&acc)[4][BM * WN / 64]) {
  using SA = GemmStage<BM, KT, A_KC>;
  using SB = GemmStage<64 * WN, KT, B_KC>;
  constexpr int MT = BM * WN / 64;  // 16-row m tiles per wave
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lq = lane & 15, gq = lane >> 4;
  const int wn = wave % WN, wm = wave / WN;
#pragma unroll
  for (int ks = 0; ks < KT; ks += 16) {
    float bvals[4][4], avals[MT][4];
    SB::template fetch<4>(Bs, 64 * wn, ks, lq, gq, bvals);
    SA::template fetch<MT>(As, 16 * MT * wm, ks, lq, gq, avals);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma4(bvals[nt][e], avals[mt][e], acc[nt][mt]);
      }
    }
  }
}

// Bias gradient of the weight-gradient GEMM: the per-thread row sums rs (rows
// 4*(tid % (BM/4)) .. +3 of the block's A tile) added over the threads in
// increasing tid order through LDS (red: >= 1024 floats, free of other use),
// written by the blocks of the first column tile.
template <int BM, bool PARTIAL>
__device__ __forceinline__ void gemm_rowsum_store(const GemmArgs& g, const float4& rs, int m0, int bt,
                                                  float* red_lds) {
  if ((PARTIAL ? g.rowsum_part : g.rowsum) == nullptr) return;
  // rows rc..rc+3 (rc = 4*(tid % R4)) are summed by the 256/R4 threads tid % R4 == rc/4
  constexpr int R4 = BM / 4;
  const int tid = threadIdx.x;
  float4* red = reinterpret_cast<float4*>(red_lds);
  __syncthreads();
  red[tid] = rs;
  __syncthreads();
  if (tid < R4) {
    float4 t = red[tid];
    for (int j = 1; j < 256 / R4; ++j) {
      const float4 u = red[tid + R4 * j];
      t.x += u.x;
      t.y += u.y;
      t.z += u.z;
      t.w += u.w;
    }
    float* dst = PARTIAL ? g.rowsum_part + (int64_t)blockIdx.z * g.M : g.rowsum + bt * g.rowsum_sb;
    const int m = m0 + 4 * tid;
    if (m + 0 < g.M) dst[m + 0] = t.x;
    if (m + 1 < g.M) dst[m + 1] = t.y;
    if (m + 2 < g.M) dst[m + 2] = t.z;
    if (m + 3 < g.M) dst[m + 3] = t.w;
  }
}

// Epilogue: acc[nt][mt] of each wave to C (bias, accumulate, split-K partials).
template <int BM, int WN, bool A_KC, bool B_KC, bool PARTIAL>
__device__ __forceinline__ void gemm_store(const GemmArgs& g, const floatx4 (&acc)[4][BM * WN / 64], int m0, int n0,
                                           int bt) {
  using SA = GemmStage<BM, 16, A_KC>;
  constexpr int MT = BM * WN / 64;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int lq = lane & 15, gq = lane >> 4;
  const int wn = wave % WN, wm = wave / WN;
  // acc[nt][mt][i] = C[m][n] with m = m0 + 16*MT*wm + SA::row_of(mt, lq) and
  // n = n0 + 64wn + SB::row_of(nt, 4gq + i): four consecutive n over i (B_KC)
  // or over nt (otherwise) go out as one 128-bit store.
  const bool vec = PARTIAL ? (g.N % 4 == 0) : g.c_vec;
  const float* bias = (!PARTIAL && g.bias != nullptr) ? g.bias + bt * g.bias_sb : nullptr;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = m0 + 16 * MT * wm + SA::row_of(mt, lq, MT);
    if (m >= g.M) continue;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // B_KC: u = nt, the vector runs over i; otherwise u = i, the vector runs over nt
      const int n = B_KC ? n0 + 64 * wn + 16 * u + 4 * gq : n0 + 64 * wn + 4 * (4 * gq + u);
      if (n >= g.N) continue;
      float4 r = B_KC ? make_float4(acc[u][mt][0], acc[u][mt][1], acc[u][mt][2], acc[u][mt][3])
                      : make_float4(acc[0][mt][u], acc[1][mt][u], acc[2][mt][u], acc[3][mt][u]);
      float* dst;
      if (PARTIAL) {
        dst = g.c + ((int64_t)blockIdx.z * g.M + m) * g.N + n;
      } else {
        dst = g.c + bt * g.c_sb + (int64_t)m * g.ldc + n;
        if (bias != nullptr) {
          r.x = (n + 0 < g.N ? bias[n + 0] : 0.f) + r.x;
          r.y = (n + 1 < g.N ? bias[n + 1] : 0.f) + r.y;
          r.z = (n + 2 < g.N ? bias[n + 2] : 0.f) + r.z;
          r.w = (n + 3 < g.N ? bias[n + 3] : 0.f) + r.w;
        }
        if (g.accumulate) {
          if (vec && n + 3 < g.N) {
            const float4 o = *reinterpret_cast<const float4*>(dst);
            r.x += o.x;
            r.y += o.y;
            r.z += o.z;
            r.w += o.w;
          } else {
            r.x += dst[0];
            if (n + 1 < g.N) r.y += dst[1];
            if (n + 2 < g.N) r.z += dst[2];
            if (n + 3 < g.N) r.w += dst[3];
          }
        }
      }
      if (vec && n + 3 < g.N) {
        *reinterpret_cast<float4*>(dst) = r;
      } else {
        dst[0] = r.x;
        if (n + 1 < g.N) dst[1] = r.y;
        if (n + 2 < g.N) dst[2] = r.z;
        if (n + 3 < g.N) dst[3] = r.w;
      }
    }
  }
}

// k loop of one output tile.  The nfull k-full stages run with stage s+1
// loaded into registers while stage s is multiplied out of LDS; the loop body
// has no branch around its loads (the last iteration reloads the final stage),
// so the loaded registers need no merge copies and the loads stay in flight
// across the MFMA work.  A partial stage at the end of the k range follows on
// its own.  FA / FB: the block's A / B rows are all in bounds and 16-byte
// aligned, so their k-full stages load unpredicated.
template <int BM, int KT, int WN, bool A_KC, bool B_KC, bool FA, bool FB>
__device__ __forceinline__ void gemm_mainloop(const GemmArgs& g, const float* A,
                                              const float* Bm, int m0, int n0, int k_begin,
                                              int k_end, float* As, float* Bs,
                                              floatx4 (&acc)[4][BM * WN / 64], float4& rs) {
  using SA = GemmStage<BM, KT, A_KC>;
  using SB = GemmStage<64 * WN, KT, B_KC>;
  const int tid = threadIdx.x;
  const int nfull = k_end > k_begin ? (k_end - k_begin) / KT : 0;
  SA sa;
  SB sb;
  if (nfull > 0) {
    sa.template load<FA>(A, g.a_sm, g.a_sk, m0, g.M, k_begin, k_end, tid);
    sb.template load<FB>(Bm, g.b_sn, g.b_sk, n0, g.N, k_begin, k_end, tid);
  }
  for (int i = 0; i < nfull; ++i) {
    __syncthreads();
    sa.store(As, tid);
    sb.store(Bs, tid);
    if (!A_KC) sa.add_to(rs);
    __syncthreads();
    const int kn = k_begin + min(i + 1, nfull - 1) * KT;
    sa.template load<FA>(A, g.a_sm, g.a_sk, m0, g.M, kn, k_end, tid);
    sb.template load<FB>(Bm, g.b_sn, g.b_sk, n0, g.N, kn, k_end, tid);
    // Memory clobber: keeps these loads here instead of letting the optimizer
    // merge them with the prologue's into one load after the loop-header phi,
    // right before the LDS store that waits for it.
    asm volatile("" ::: "memory");
    gemm_stage_mfma<BM, KT, WN, A_KC, B_KC>(As, Bs, acc);
  }
  const int kp = k_begin + nfull * KT;
  if (kp < k_end) {
    sa.template load<false>(A, g.a_sm, g.a_sk, m0, g.M, kp, k_end, tid);
    sb.template load<false>(Bm, g.b_sn, g.b_sk, n0, g.N, kp, k_end, tid);
    __syncthreads();
    sa.store(As, tid);
    sb.store(Bs, tid);
    if (!A_KC) sa.add_to(rs);
    __syncthreads();
    gemm_stage_mfma<BM, KT, WN, A_KC, B_KC>(As, Bs, acc);
  }
}

// BM x 64*WN output tile per 256-thread block, (4/WN) x WN waves of
// (BM*WN/4) x 64, KT-deep k stages.  MFMA rows are output columns n, MFMA
// columns output rows m.
template <int BM, int KT, int WN, bool A_KC, bool B_KC, bool PARTIAL>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs g) {
  constexpr int BN = 64 * WN;
  using SA = GemmStage<BM, KT, A_KC>;
  using SB = GemmStage<BN, KT, B_KC>;
  constexpr int MT = BM * WN / 64;  // 16-row m tiles per wave
  __shared__ __align__(16) float As[SA::ELEMS];
  __shared__ __align__(16) float Bs[SB::ELEMS];
  // XCD-aware tile order: blocks are dealt round-robin to the 8 XCDs by linear
  // id, so when a split's tile count is a multiple of 8, block j of XCD x takes
  // tile x*(tiles/8) + j: each XCD then sweeps a contiguous band of m-tiles
  // across all n-tiles and reuses the band's A rows from its own L2.
  int tile = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  const int tiles = (int)(gridDim.x * gridDim.y);
  if (tiles % 8 == 0) tile = (tile % 8) * (tiles / 8) + tile / 8;
  const int n0 = (tile % (int)gridDim.x) * BN, m0 = (tile / (int)gridDim.x) * BM;
  const int bt = (int)blockIdx.z / g.splits;
  const int k_begin = ((int)blockIdx.z % g.splits) * g.k_chunk;
  const float* A = g.a + bt * g.a_sb;
  const float* Bm = g.b + bt * g.b_sb;
  const int k_end = min(g.K, k_begin + g.k_chunk);

  floatx4 acc[4][MT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Interior blocks take unpredicated loads for every k stage but a partial last one.
  const bool fa = g.a_vec && m0 + BM <= g.M;
  const bool fb = g.b_vec && n0 + BN <= g.N;
  float4 rs = make_float4(0.f, 0.f, 0.f, 0.f);
  if (fa && fb)
    gemm_mainloop<BM, KT, WN, A_KC, B_KC, true, true>(g, A, Bm, m0, n0, k_begin, k_end, As, Bs, acc, rs);
  else if (fa)
    gemm_mainloop<BM, KT, WN, A_KC, B_KC, true, false>(g, A, Bm, m0, n0, k_begin, k_end, As, Bs, acc, rs);
  else if (fb)
    gemm_mainloop<BM, KT, WN, A_KC, B_KC, false, true>(g, A, Bm, m0, n0, k_begin, k_end, As, Bs, acc, rs);
  else
    gemm_mainloop<BM, KT, WN, A_KC, B_KC, false, false>(g, A, Bm, m0, n0, k_begin, k_end, As, Bs, acc, rs);

  static_assert(SA::ELEMS >= 4 * 256, "the row-sum exchange fits in the A stage");
  if (!A_KC && n0 == 0) gemm_rowsum_store<BM, PARTIAL>(g, rs, m0, bt, As);  // As is free after the k loop
  gemm_store<BM, WN, A_KC, B_KC, PARTIAL>(g, acc, m0, n0, bt);
}

// ---------------------------------------------------------------- direct-to-LDS stages
// gemm_kernel's k loop with each stage fetched by global_load_lds (global ->
// LDS, no staging registers) into one of two LDS buffers: one barrier per
// stage, and the next stage in flight while the current one is multiplied.
// Stage layouts are unpadded, so that one 64-lane DMA instruction fills 64
// consecutive quads: a k-contiguous operand is [ROWS][KT] with quad c of row
// r stored at quad c ^ gemm_swz<KT>(r) -- conflict-free 128-bit reads for the
// fetch pattern (lane (lq, g) reads quad ks/4 + g of row 16t + lq), checked
// against the lane grouping measured for ds_read_b128 -- and a row-contiguous
// operand is [KT][ROWS] (a lane reads quad lq of one k-row: no swizzle
// needed).  Rows past the operand's extent read its last row (quad) and only
// feed outputs that are never stored; k past the block's range reads a zero
// quad.  Requires 16-byte aligned rows, K % 4 == 0 and, for a row-contiguous
// operand, an extent that is a multiple of 4 (gemm_dma_ok).  Serves all three
// projection GEMMs; for the weight gradient the bias row sums are read from
// the staged A tiles.

template <int KT>
__device__ __forceinline__ int gemm_swz(int r) {
  return KT == 16 ? (r >> 1) & 3 : (((r >> 1) & 1) << 2) | (((r >> 2) & 1) << 1);
}

template <int ROWS, int KT, bool KC>
struct DmaStage {
  static constexpr int QUADS = ROWS * KT / 4;
  static constexpr int IPW = QUADS / 256;  // DMA instructions per wave and stage (four waves)
  static_assert(QUADS % 256 == 0, "a stage must split evenly over four waves");
  uint32_t off[IPW];  // byte offset of this lane's source quad for k0 = 0 (< 2 GiB: gemm_dma_ok)
  int kq[IPW];        // k of that quad's first element within the stage
  // rows r0.. of the operand (extent R), element (r, k) at p[r*s_r + k*s_k]
  __device__ __forceinline__ void init(int64_t s_r, int64_t s_k, int r0, int R, int wave, int lane) {
#pragma unroll
    for (int u = 0; u < IPW; ++u) {
      const int p = 64 * (IPW * wave + u) + lane;  // the LDS quad this lane fills
      if (KC) {
        const int row = p / (KT / 4);
        const int c = (p % (KT / 4)) ^ gemm_swz<KT>(row);
        off[u] = (uint32_t)(((int64_t)min(r0 + row, R - 1) * s_r + 4 * c) * 4);
        kq[u] = 4 * c;
      } else {
        const int kr = p / (ROWS / 4), rq = p % (ROWS / 4);
        off[u] = (uint32_t)(((int64_t)kr * s_k + min(r0 + 4 * rq, R - 4)) * 4);
        kq[u] = kr;
      }
    }
  }
  // The stage at k0.  A stage wholly inside [.., k_end) is fetched with buffer
  // loads: the operand's descriptor and the stage's byte offset k0*s_k*4 are
  // wave-uniform (scalar registers), each lane adds its fixed offset, so the
  // issue needs no per-lane address arithmetic.  A stage that reaches past
  // k_end forms per-lane addresses and fetches the zero quad past it.
  __device__ __forceinline__ void issue(__amdgpu_buffer_rsrc_t rsrc, const float* base, int64_t s_k, int k0,
                                        int k_end, float* lds, int wave) const {
    if (k0 + KT <= k_end) {
      const int soff = (int)((int64_t)k0 * s_k * 4);
#pragma unroll
      for (int u = 0; u < IPW; ++u)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc, (__attribute__((address_space(3))) void*)(lds + 256 * (IPW * wave + u)), 16, (int)off[u], soff,
            0, 0);
    } else {
      const char* b0 = reinterpret_cast<const char*>(base + (int64_t)k0 * s_k);
#pragma unroll
      for (int u = 0; u < IPW; ++u) {
        const float* src = k0 + kq[u] < k_end ? reinterpret_cast<const float*>(b0 + off[u]) : g_zero_quad;
        dma_quad(src, lds + 256 * (IPW * wave + u));
      }
    }
  }
  // The MFMA operands of GemmStage::fetch from this layout (same tile and
  // lane mapping, so the same epilogue).
  template <int TPW>
  __device__ __forceinline__ static void fetch(const float* lds, int rowbase, int ks, int lq, int g,
                                               float (&out)[TPW][4]) {
    if (KC) {
#pragma unroll
      for (int t = 0; t < TPW; ++t) {
        const int row = rowbase + 16 * t + lq;
        const float4 x = *reinterpret_cast<const float4*>(&lds[row * KT + 4 * ((ks / 4 + g) ^ gemm_swz<KT>(row))]);
        out[t][0] = x.x;
        out[t][1] = x.y;
        out[t][2] = x.z;
        out[t][3] = x.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float* src = &lds[(ks + 4 * g + e) * ROWS + rowbase + TPW * lq];
        if (TPW == 4) {
          const float4 x = *reinterpret_cast<const float4*>(src);
          out[0][e] = x.x;
          out[1 % TPW][e] = x.y;
          out[2 % TPW][e] = x.z;
          out[3 % TPW][e] = x.w;
        } else {
#pragma unroll
          for (int t = 0; t < TPW; ++t) out[t][e] = src[t];
        }
      }
    }
  }
};

template <int BM, int KT, int WN, bool A_KC, bool B_KC, bool PARTIAL>
__global__ __launch_bounds__(256) void gemm_dma_kernel(GemmArgs g) {
  constexpr int BN = 64 * WN;
  constexpr int MT = BM * WN / 64;  // 16-row m tiles per wave
  using DA = DmaStage<BM, KT, A_KC>;
  using DB = DmaStage<BN, KT, B_KC>;
  __shared__ __align__(16) float As0[BM * KT];
  __shared__ __align__(16) float As1[BM * KT];
  __shared__ __align__(16) float Bs0[BN * KT];
  __shared__ __align__(16) float Bs1[BN * KT];
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int lq = lane & 15, gq = lane >> 4;
  const int wn = wave % WN, wm = wave / WN;
  // tile order as in gemm_kernel (XCD-aware)
  int tile = (int)(blockIdx.y * gridDim.x + blockIdx.x);
  const int tiles = (int)(gridDim.x * gridDim.y);
  if (tiles % 8 == 0) tile = (tile % 8) * (tiles / 8) + tile / 8;
  const int n0 = (tile % (int)gridDim.x) * BN, m0 = (tile / (int)gridDim.x) * BM;
  const int bt = (int)blockIdx.z / g.splits;
  const int k_begin = ((int)blockIdx.z % g.splits) * g.k_chunk;
  const float* A = g.a + bt * g.a_sb;
  const float* Bm = g.b + bt * g.b_sb;
  const int k_end = min(g.K, k_begin + g.k_chunk);

  DA da;
  DB db;
  da.init(g.a_sm, g.a_sk, m0, g.M, wave, lane);
  db.init(g.b_sn, g.b_sk, n0, g.N, wave, lane);
  // buffer descriptors over each operand's extent (raw, 32-bit records)
  const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(A, g.a_bytes);
  const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(Bm, g.b_bytes);

  floatx4 acc[4][MT];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < MT; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

  const int nst = k_end > k_begin ? (k_end - k_begin + KT - 1) / KT : 0;
  auto issue = [&](int s, float* Ad, float* Bd) {
    const int k0 = k_begin + s * KT;
    da.issue(ra, A, g.a_sk, k0, k_end, Ad, wave);
    db.issue(rb, Bm, g.b_sk, k0, k_end, Bd, wave);
  };
  // bias gradient (row-contiguous A, the weight-gradient GEMM): the blocks of
  // the first column tile add up the staged A rows, each thread rows
  // 4*(tid % (BM/4)) .. +3 over every (256/(BM/4))-th k row of a stage -- the
  // per-thread sums gemm_rowsum_store reduces
  const bool want_rs = !A_KC && n0 == 0 && (PARTIAL ? g.rowsum_part : g.rowsum) != nullptr;
  float4 rs = make_float4(0.f, 0.f, 0.f, 0.f);
  auto step = [&](int s, const float* Ac, const float* Bc, float* An, float* Bn) {
    wait_vmem();
    __syncthreads();  // stage s is in LDS; every wave is done with stage s - 1
    if (s + 1 < nst) issue(s + 1, An, Bn);
    if constexpr (!A_KC) {
      if (want_rs) {
        constexpr int R4 = BM / 4, KSTEP = 256 / R4;
        const int tid = threadIdx.x;
#pragma unroll
        for (int kr = tid / R4; kr < KT; kr += KSTEP) {
          const float4 x = *reinterpret_cast<const float4*>(&Ac[kr * BM + 4 * (tid % R4)]);
          rs.x += x.x;
          rs.y += x.y;
          rs.z += x.z;
          rs.w += x.w;
        }
      }
    }
#pragma unroll
    for (int ks = 0; ks < KT; ks += 16) {
      float bvals[4][4], avals[MT][4];
      DB::template fetch<4>(Bc, 64 * wn, ks, lq, gq, bvals);
      DA::template fetch<MT>(Ac, 16 * MT * wm, ks, lq, gq, avals);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) {
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = mfma4(bvals[nt][e], avals[mt][e], acc[nt][mt]);
        }
      }
    }
  };
  if (nst > 0) issue(0, As0, Bs0);
  for (int s = 0; s < nst; s += 2) {
    step(s, As0, Bs0, As1, Bs1);
    if (s + 1 < nst) step(s + 1, As1, Bs1, As0, Bs0);
  }

  static_assert(BM * KT >= 4 * 256, "the row-sum exchange fits in an A stage");
  if (!A_KC && n0 == 0) gemm_rowsum_store<BM, PARTIAL>(g, rs, m0, bt, As0);  // after its own barrier
  gemm_store<BM, WN, A_KC, B_KC, PARTIAL>(g, acc, m0, n0, bt);
}

// C[bt][m][n] (+)= bias[bt][n] + sum_s part[bt*splits + s][m][n], s in increasing order.
// W consecutive n per thread (W = 4 when N % 4 == 0: 128-bit loads); the
// partials are loaded eight splits at a time, then added in split order.
template <int W>
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float* __restrict__ part, GemmArgs g) {
  const int64_t MN = (int64_t)g.M * g.N;
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * W;
  if (i >= MN * g.batch) return;
  const int bt = (int)(i / MN);
  const int64_t e = i - bt * MN;
  const int m = (int)(e / g.N), n = (int)(e % g.N);
  const float* src = part + (int64_t)bt * g.splits * MN + e;
  float s[W];
#pragma unroll
  for (int w = 0; w < W; ++w) s[w] = 0.f;
  for (int z0 = 0; z0 < g.splits; z0 += 8) {
    float v[8][W];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const bool in = z0 + u < g.splits;
      const float* p = src + (int64_t)(in ? z0 + u : 0) * MN;
      if (W == 4) {
        const float4 x = *reinterpret_cast<const float4*>(p);
        v[u][0] = x.x;
        v[u][1 % W] = x.y;
        v[u][2 % W] = x.z;
        v[u][3 % W] = x.w;
      } else {
        v[u][0] = p[0];
      }
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      if (z0 + u < g.splits) {
#pragma unroll
        for (int w = 0; w < W; ++w) s[w] += v[u][w];
      }
    }
  }
  float* dst = g.c + bt * g.c_sb + (int64_t)m * g.ldc + n;
  float r[W];
#pragma unroll
  for (int w = 0; w < W; ++w) {
    r[w] = (g.bias != nullptr ? g.bias[bt * g.bias_sb + n + w] : 0.f) + s[w];
    if (g.accumulate) r[w] = dst[w] + r[w];
  }
  if (W == 4 && g.c_vec) {
    *reinterpret_cast<float4*>(dst) = make_float4(r[0], r[1 % W], r[2 % W], r[3 % W]);
  } else {
#pragma unroll
    for (int w = 0; w < W; ++w) dst[w] = r[w];
  }
  if (n == 0 && g.rowsum != nullptr) {
    const float* rp = g.rowsum_part + (int64_t)bt * g.splits * g.M + m;
    float t = 0.f;
    for (int z0 = 0; z0 < g.splits; z0 += 8) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = rp[(int64_t)(z0 + u < g.splits ? z0 + u : 0) * g.M];
#pragma unroll
      for (int u = 0; u < 8; ++u)
        if (z0 + u < g.splits) t += v[u];
    }
    g.rowsum[bt * g.rowsum_sb + m] = t;
  }
}

namespace {

// Output tile: the largest of 128 x 128, 64 x 128 that gives at least eight
// blocks per CU; 64-column tiles when N <= 64, and for N <= 256 when 64 x 128
// tiles would leave CUs with fewer (same padding, twice the blocks).  Split-K
// then picks its factor by rounds of resident blocks (gemm_splits; it once
// aimed for 1024 blocks in powers of two: weight gradients of the layer step
// 343 -> 328 us, of the wave step 174 -> 166 us with the rounds model).  Both thresholds were swept on the layer and wave
// steps (tile 256/512/1024 blocks x split 512/1024/2048: 1024/1024 best, layer
// 1.465 vs 1.501 ms at 512/512, wave 0.865 vs 0.877 ms); with the buffer-load
// stages the tile threshold moved to 2048 (the 2304 x 768 c_attn forward in
// 64 x 128 tiles, three full rounds of three blocks per CU: 126 vs 111 TFLOP/s,
// layer step 1.369 vs 1.400 ms).
constexpr int kCUs = 256;
#ifndef WHA_GEMM_TILE_BLOCKS
#define WHA_GEMM_TILE_BLOCKS (8 * kCUs)
#endif
struct GemmTile {
  int bm, bn;
};
GemmTile gemm_tile(int M, int N, int batch) {
  auto blocks = [&](int bm, int bn) { return (int64_t)((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
  if (N <= 64) return {blocks(128, 64) >= WHA_GEMM_TILE_BLOCKS ? 128 : 64, 64};
  if (blocks(128, kGBN) >= WHA_GEMM_TILE_BLOCKS) return {128, kGBN};
  if (blocks(64, kGBN) >= WHA_GEMM_TILE_BLOCKS || N > 256) return {64, kGBN};
  return {64, 64};
}

#ifndef WHA_GEMM_FIXK
#define WHA_GEMM_FIXK 128
#endif
// Split-K factor: the split count that minimises rounds x (k per split + a fixed
// per-block cost), where a round is one block per slot (blocks a CU holds at
// once: 2 for 128 x 128 tiles, 3 for 64 x 128, 5 for 64 x 64, by their VGPRs
// and LDS), keeping >= min_k k per split.
int gemm_splits(int M, int N, int K, int batch, int min_k = 256) {
  const GemmTile t = gemm_tile(M, N, batch);
  const int64_t tiles = (int64_t)((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn) * batch;
  const int64_t slots = (int64_t)kCUs * (t.bn == 64 ? 5 : t.bm == 128 ? 2 : 3);
  int best = 1;
  int64_t best_cost = INT64_MAX;
  for (int s = 1; s <= 32; ++s) {
    if (s > 1 && K / s < min_k) break;
    const int64_t rounds = (tiles * s + slots - 1) / slots;
    const int64_t cost = rounds * ((K + s - 1) / s + WHA_GEMM_FIXK);
    if (cost < best_cost) {
      best_cost = cost;
      best = s;
    }
  }
  return best;
}


// The direct-to-LDS kernel serves y = x W^T + b, dx = dy W and dW = dy^T x
// (measured at M = 8192 with per-lane global addresses: layer step 1.477 vs
// 1.507 ms, the c_attn forward 106 vs 91 TFLOP/s, and the weight gradient
// slower than register-staged stages; with buffer loads: 768 x 768 forward /
// dx / dW 107 / 116 / 95 TFLOP/s against 95 / 107 / 91, 2304 x 768 dW 122
// against 111, layer step 1.339 vs 1.460 ms) when every row is 16-byte aligned
// along its operand's contiguous direction (a_vec, b_vec), K % 4 == 0, a
// row-contiguous operand has a multiple-of-4 extent and each operand spans
// less than 2 GiB.  Otherwise gemm_kernel (register-staged stages) runs.
template <bool A_KC, bool B_KC>
bool gemm_dma_ok(GemmArgs& g) {
  if (!(WHA_GEMM_DMA && g.a_vec && g.b_vec && g.K % 4 == 0 && (A_KC || g.M % 4 == 0) &&
        (B_KC || g.N % 4 == 0)))
    return false;
  // DmaStage keeps 32-bit byte offsets and buffer extents: each operand's
  // reachable extent (one batch) must stay below 2 GiB
  const int64_t a_ext = 4 * (A_KC ? (int64_t)(g.M - 1) * g.a_sm + g.K : (int64_t)(g.K - 1) * g.a_sk + g.M);
  const int64_t b_ext = 4 * (B_KC ? (int64_t)(g.N - 1) * g.b_sn + g.K : (int64_t)(g.K - 1) * g.b_sk + g.N);
  if (a_ext >= ((int64_t)1 << 31) || b_ext >= ((int64_t)1 << 31)) return false;
  g.a_bytes = (uint32_t)a_ext;
  g.b_bytes = (uint32_t)b_ext;
  return true;
}

template <int BM, int KT, int WN, bool A_KC, bool B_KC>
hipError_t gemm_launch(GemmArgs g, float* ws, int splits, const char* name, hipStream_t stream) {
  const dim3 grid((g.N + 64 * WN - 1) / (64 * WN), (g.M + BM - 1) / BM, splits * g.batch);
  g.splits = splits;
  const bool dma = gemm_dma_ok<A_KC, B_KC>(g);
  constexpr int KD = WHA_GEMM_DMA_KT;
  TimingScope ts(name, stream);
  if (splits == 1) {
    g.k_chunk = dma ? ((g.K + KD - 1) / KD) * KD : ((g.K + KT - 1) / KT) * KT;
    if (dma) {
      hipLaunchKernelGGL((gemm_dma_kernel<BM, KD, WN, A_KC, B_KC, false>), grid, dim3(256), 0, stream, g);
      return hipGetLastError();
    }
    hipLaunchKernelGGL((gemm_kernel<BM, KT, WN, A_KC, B_KC, false>), grid, dim3(256), 0, stream, g);
    return hipGetLastError();
  }
  const int per = (g.K + splits - 1) / splits;
  GemmArgs p = g;
  p.k_chunk = dma ? ((per + KD - 1) / KD) * KD : ((per + KT - 1) / KT) * KT;
  p.c = ws;
  p.bias = nullptr;
  if (dma)
    hipLaunchKernelGGL((gemm_dma_kernel<BM, KD, WN, A_KC, B_KC, true>), grid, dim3(256), 0, stream, p);
  else
    hipLaunchKernelGGL((gemm_kernel<BM, KT, WN, A_KC, B_KC, true>), grid, dim3(256), 0, stream, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int64_t total = (int64_t)g.M * g.N * g.batch;
  if (g.N % 4 == 0)
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel<4>, dim3((unsigned)((total / 4 + 255) / 256)), dim3(256), 0,
                       stream, (const float*)ws, g);
  else
    hipLaunchKernelGGL(gemm_splitk_reduce_kernel<1>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                       (const float*)ws, g);
  return hipGetLastError();
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ---------------------------------------------------------------- 64 x 64 per-head projections
// The per-head projections of 64-wide heads (the wave attention's value
// projection and its input gradient): for head bt,
//   out[m][j] (+)= sum_i A[m][i] Wop(i, j) (+ bias[j]),   i, j < 64,
// with Wop(i, j) = W_bt[j][i] (TRANS_W: y = x W^T + b) or W_bt[i][j]
// (dx += dy W).  K = N = 64 leaves the generic tiles two k stages, so their
// time goes to prologues and epilogues.  Here each wave holds the head's
// operand in registers -- lane (lq, g) keeps Wop(i, 4lq + nt) for its 16
// contraction indices i = 16u + 4g + e, MFMA k-step 4u + e, so every MFMA sums
// the same four products, in the same step order, as gemm_dma_kernel's
// (results bit-identical to it); MFMA column lq of n-tile nt is output column
// 4lq + nt; the block stages the operand once in LDS -- and streams 16-row tiles: four 128-bit loads of a row's floats
// 16u + 4g .. +3 per lane (the next tile's issued before the current tile's 64
// MFMAs), four 128-bit stores of whole 64-float rows per lane.  Memory-bound.
constexpr int kHead64Waves = 4;
constexpr int kHead64TilesPerWave = 2;

template <bool TRANS_W, bool ACC>
__global__ __launch_bounds__(256) void head64_gemm_kernel(const float* __restrict__ A, int64_t lda, int64_t a_sb,
                                                          const float* __restrict__ W, int64_t w_sb,
                                                          const float* __restrict__ bias, int64_t b_sb,
                                                          float* __restrict__ C, int64_t ldc, int64_t c_sb, int M) {
  const int bt = blockIdx.y;
  const int lane = threadIdx.x & 63, lq = lane & 15, g = lane >> 4;
  const int wave = threadIdx.x >> 6;
  const float* Ab = A + (int64_t)bt * a_sb;
  const float* Wb = W + (int64_t)bt * w_sb;
  float* Cb = C + (int64_t)bt * c_sb;

  // the head's operand through LDS (one 16 KB load per block): Ws[i * 64 + j] = Wop(i, j)
  __shared__ __align__(16) float Ws[64 * 64];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const int q = (int)threadIdx.x + 256 * p;  // quad q of W: row q / 16, floats 4 (q % 16) .. +3
    const int r = q >> 4, c4 = 4 * (q & 15);
    const float4 v = *reinterpret_cast<const float4*>(Wb + r * 64 + c4);
    if constexpr (TRANS_W) {
      Ws[(c4 + 0) * 64 + r] = v.x;
      Ws[(c4 + 1) * 64 + r] = v.y;
      Ws[(c4 + 2) * 64 + r] = v.z;
      Ws[(c4 + 3) * 64 + r] = v.w;
    } else {
      *reinterpret_cast<float4*>(&Ws[r * 64 + c4]) = v;
    }
  }
  __syncthreads();
  // wop[nt][4u + e] = Wop(16u + 4g + e, 4lq + nt): one 128-bit read of quad lq of
  // row 16u + 4g + e per k-step (each 16-lane set reads 16 different quads)
  float wop[4][16];
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const float4 v = *reinterpret_cast<const float4*>(&Ws[(16 * (s >> 2) + 4 * g + (s & 3)) * 64 + 4 * lq]);
    wop[0][s] = v.x;
    wop[1][s] = v.y;
    wop[2][s] = v.z;
    wop[3][s] = v.w;
  }
  const float4 bv = (!ACC && bias != nullptr) ? *reinterpret_cast<const float4*>(bias + (int64_t)bt * b_sb + 4 * lq)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);

  const int n_tiles = (M + 15) / 16;
  const int stride = (int)gridDim.x * kHead64Waves;
  // this lane's part of tile t: a[4u + e] = float 16u + 4g + e of row 16t + lq (zeros past M)
  auto load_a = [&](int t, float (&a)[16]) {
    const int r = 16 * t + lq;
    const bool ok = t < n_tiles && r < M;
    const float* p = Ab + (int64_t)(ok ? r : 0) * lda + 4 * g;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float4 v = *reinterpret_cast<const float4*>(p + 16 * u);
      a[4 * u + 0] = ok ? v.x : 0.f;
      a[4 * u + 1] = ok ? v.y : 0.f;
      a[4 * u + 2] = ok ? v.z : 0.f;
      a[4 * u + 3] = ok ? v.w : 0.f;
    }
  };
  int t = (int)blockIdx.x * kHead64Waves + wave;
  float a_cur[16], a_nxt[16];
  load_a(t, a_cur);
  for (; t < n_tiles; t += stride) {
    load_a(t + stride, a_nxt);
    // lane results: rows 16t + 4g + i, columns 4lq .. 4lq + 3
    float4 prev[4];
    if constexpr (ACC) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 16 * t + 4 * g + i;
        prev[i] = r < M ? *reinterpret_cast<const float4*>(Cb + (int64_t)r * ldc + 4 * lq)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    floatx4 acc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) acc[nt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 16; ++s) {
#pragma unroll
      for (int nt = 0; nt < 4; ++nt) acc[nt] = mfma4(a_cur[s], wop[nt][s], acc[nt]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = 16 * t + 4 * g + i;
      if (r >= M) continue;
      float4 o = make_float4(acc[0][i], acc[1][i], acc[2][i], acc[3][i]);
      const float4 add = ACC ? prev[i] : bv;
      o.x += add.x;
      o.y += add.y;
      o.z += add.z;
      o.w += add.w;
      *reinterpret_cast<float4*>(Cb + (int64_t)r * ldc + 4 * lq) = o;
    }
#pragma unroll
    for (int e = 0; e < 16; ++e) a_cur[e] = a_nxt[e];
  }
}

// Whether head64_gemm_kernel serves a batched projection: 64 x 64 per head,
// every pointer, row stride and batch stride 16-byte aligned.
bool head64_ok(const float* a, int64_t lda, int64_t a_sb, const float* w, int64_t w_sb, const float* b,
               int64_t b_sb, const float* c, int64_t ldc, int64_t c_sb, int M, int N, int K, int batch) {
  return WHA_HEAD64 && N == 64 && K == 64 && M > 0 && batch > 0 && batch <= 65535 && aligned16(a) && aligned16(w) &&
         aligned16(c) && (b == nullptr || (aligned16(b) && b_sb % 4 == 0)) && lda % 4 == 0 && a_sb % 4 == 0 &&
         w_sb % 4 == 0 && ldc % 4 == 0 && c_sb % 4 == 0;
}

template <bool TRANS_W, bool ACC>
hipError_t head64_launch(const float* a, int64_t lda, int64_t a_sb, const float* w, int64_t w_sb, const float* b,
                         int64_t b_sb, float* c, int64_t ldc, int64_t c_sb, int M, int batch, const char* name,
                         hipStream_t stream) {
  const int n_tiles = (M + 15) / 16;
  const int per_block = kHead64Waves * kHead64TilesPerWave;
  const int gx = std::min((n_tiles + per_block - 1) / per_block, 65535);
  TimingScope ts(name, stream);
  hipLaunchKernelGGL((head64_gemm_kernel<TRANS_W, ACC>), dim3((unsigned)gx, (unsigned)batch), dim3(256), 0, stream,
                     a, lda, a_sb, w, w_sb, b, b_sb, c, ldc, c_sb, M);
  return hipGetLastError();
}

template <bool A_KC, bool B_KC>
hipError_t gemm_t(GemmArgs g, float* ws, const char* name, hipStream_t stream, int min_k = 256) {
  const int splits = ws ? gemm_splits(g.M, g.N, g.K, g.batch, min_k) : 1;
  // 128-bit loads need every row start along the contiguous direction 16-byte aligned
  g.a_vec = aligned16(g.a) && g.a_sb % 4 == 0 && (A_KC ? g.a_sm % 4 == 0 : g.a_sk % 4 == 0);
  g.b_vec = aligned16(g.b) && g.b_sb % 4 == 0 && (B_KC ? g.b_sn % 4 == 0 : g.b_sk % 4 == 0);
  const GemmTile t = gemm_tile(g.M, g.N, g.batch);
  const bool bm128 = t.bm == 128;
  if (t.bn == 64)
    return bm128 ? gemm_launch<128, WHA_GEMM_KT, 1, A_KC, B_KC>(g, ws, splits, name, stream)
                 : gemm_launch<64, WHA_GEMM_KT, 1, A_KC, B_KC>(g, ws, splits, name, stream);
  return bm128 ? gemm_launch<128, WHA_GEMM_KT, 2, A_KC, B_KC>(g, ws, splits, name, stream)
               : gemm_launch<64, WHA_GEMM_KT, 2, A_KC, B_KC>(g, ws, splits, name, stream);
}

}  // namespace

size_t linear_dw_workspace_floats(int N, int K, int64_t M, int batch) {
  // split-K partials of the [batch][N][K] weight gradient and of the bias gradient
  const int splits = gemm_splits(N, K, (int)(M > 0x7fffffff ? 0x7fffffff : M), batch);
  const size_t part = splits > 1 ? (size_t)splits * batch * N * (K + 1) : 0;
  return part + 64;
}

// Few output tiles (decode-sized M): split K down to 64 per split.
constexpr int kFwdMinK = 64;

size_t linear_fwd_workspace_floats(int M, int N, int K, int batch) {
  const int splits = gemm_splits(M, N, K, batch, kFwdMinK);
  return splits > 1 ? (size_t)splits * batch * M * N : 0;
}

// y[bt] = x[bt] w[bt]^T + b[bt]:  x [M][K] (row stride ldx), w [N][K], y [M][N] (row stride ldy);
// ws (linear_fwd_workspace_floats, or nullptr for no split-K) lets few-tile shapes split K.
hipError_t launch_linear_fwd_batched(const float* x, int64_t ldx, int64_t x_sb, const float* w, int64_t w_sb,
                                     const float* b, int64_t b_sb, float* y, int64_t ldy, int64_t y_sb, int M,
                                     int N, int K, int batch, hipStream_t stream, float* ws) {
  if (head64_ok(x, ldx, x_sb, w, w_sb, b, b_sb, y, ldy, y_sb, M, N, K, batch))
    return head64_launch<true, false>(x, ldx, x_sb, w, w_sb, b, b_sb, y, ldy, y_sb, M, batch, "linear_fwd", stream);
  GemmArgs g{x, ldx, 1, w, (int64_t)K, 1, y, ldy, b, M, N, K, 0,
             aligned16(y) && ldy % 4 == 0 && y_sb % 4 == 0, false};
  g.batch = batch;
  g.a_sb = x_sb;
  g.b_sb = w_sb;
  g.c_sb = y_sb;
  g.bias_sb = b_sb;
  return gemm_t<true, true>(g, ws, "linear_fwd", stream, kFwdMinK);
}

// dx[bt] (+)= dy[bt] w[bt]:  dy [M][N], w [N][K], dx [M][K]
hipError_t launch_linear_bwd_dx_batched(const float* dy, int64_t lddy, int64_t dy_sb, const float* w,
                                        int64_t w_sb, float* dx, int64_t lddx, int64_t dx_sb, int M, int N,
                                        int K, int batch, bool accumulate, hipStream_t stream) {
  if (head64_ok(dy, lddy, dy_sb, w, w_sb, nullptr, 0, dx, lddx, dx_sb, M, N, K, batch))
    return accumulate ? head64_launch<false, true>(dy, lddy, dy_sb, w, w_sb, nullptr, 0, dx, lddx, dx_sb, M, batch,
                                                   "linear_bwd_dx", stream)
                      : head64_launch<false, false>(dy, lddy, dy_sb, w, w_sb, nullptr, 0, dx, lddx, dx_sb, M, batch,
                                                    "linear_bwd_dx", stream);
  // dx[m][k] = sum_n dy[m][n] w[n][k]: GEMM with (M, N=K_in, K=N_out)
  GemmArgs g{dy, lddy, 1, w, 1, (int64_t)K, dx, lddx, nullptr, M, K, N, 0,
             aligned16(dx) && lddx % 4 == 0 && dx_sb % 4 == 0, accumulate};
  g.batch = batch;
  g.a_sb = dy_sb;
  g.b_sb = w_sb;
  g.c_sb = dx_sb;
  return gemm_t<true, false>(g, nullptr, "linear_bwd_dx", stream);
}

// dw[bt] = dy[bt]^T x[bt] over the M rows:  dy [M][N], x [M][K], dw [N][K];
// db[bt*N + n] = sum_m dy[bt][m][n] when db != nullptr, summed inside the same GEMM (row
// sums of its A operand).  ws: linear_dw_workspace_floats.
hipError_t launch_linear_bwd_dw_batched(const float* dy, int64_t lddy, int64_t dy_sb, const float* x,
                                        int64_t ldx, int64_t x_sb, float* dw, int64_t dw_sb, float* db, int M,
                                        int N, int K, int batch, float* ws, hipStream_t stream) {
  // dw[n][k] = sum_m dy[m][n] x[m][k]: GEMM with (M=N_out, N=K_in, K=M rows), both operands
  // contiguous along the output index
  GemmArgs g{dy, 1, lddy, x, 1, ldx, dw, (int64_t)K, nullptr, N, K, M, 0,
             aligned16(dw) && K % 4 == 0 && dw_sb % 4 == 0, false};
  g.batch = batch;
  g.a_sb = dy_sb;
  g.b_sb = x_sb;
  g.c_sb = dw_sb;
  const int splits = gemm_splits(N, K, M, batch);
  float* part = splits > 1 ? ws : nullptr;
  if (db != nullptr) {
    g.rowsum = db;
    g.rowsum_sb = N;
    if (splits > 1) g.rowsum_part = ws + (size_t)splits * batch * N * K;
  }
  return gemm_t<false, false>(g, part, "linear_bwd_dw", stream);
}

size_t linear_dw_workspace_floats(int N, int K, int64_t M) { return linear_dw_workspace_floats(N, K, M, 1); }

hipError_t launch_linear_fwd(const float* x, int64_t ldx, const float* w, const float* b, float* y, int64_t ldy,
                             int M, int N, int K, hipStream_t stream) {
  return launch_linear_fwd_batched(x, ldx, 0, w, 0, b, 0, y, ldy, 0, M, N, K, 1, stream);
}

hipError_t launch_linear_bwd_dx(const float* dy, int64_t lddy, const float* w, float* dx, int64_t lddx, int M,
                                int N, int K, hipStream_t stream) {
  return launch_linear_bwd_dx_batched(dy, lddy, 0, w, 0, dx, lddx, 0, M, N, K, 1, false, stream);
}

hipError_t launch_linear_bwd_dw(const float* dy, int64_t lddy, const float* x, int64_t ldx, float* dw, float* db,
                                int M, int N, int K, float* ws, hipStream_t stream) {
  return launch_linear_bwd_dw_batched(dy, lddy, 0, x, ldx, 0, dw, 0, db, M, N, K, 1, ws, stream);
}

}  // namespace wha
