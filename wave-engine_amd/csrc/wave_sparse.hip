// Bucket-sparse wave attention core (gfx950, fp32 MFMA): the results of the
// all-pairs kernels in wave_attn.hip (the reference's wave_attention_forward /
// _backward_full core, src/common/attn.rs:167-224, math/attn_backward.rs) with
// MFMA work only where the bucket mask can admit a pair.
//
// The mask admits key k for query q (k <= q) when bucket(k) is within one of
// bucket(q) mod 8, or k = q - 1.  In position order every 16-key block holds
// almost every bucket, so the all-pairs kernels execute every causal pair and
// discard ~5/8 of them.  Here each (b,h) first sorts its positions by bucket
// (stable, so positions rise within a bucket) and gathers the operands into
// that order.  A 64-row tile of sorted queries then only meets the keys of the
// buckets next to its own -- a cyclic window of sorted indices -- and inside
// the window 16 x 16 blocks are executed only when
//   - some bucket of the query chunk is within one of some bucket of the key
//     chunk (per-chunk 8-bit bucket sets), and
//   - the key chunk's smallest position does not exceed the query chunk's
//     largest (causality),
// which is the same test from both sides, so the key-stationary dK/dV kernel
// writes exactly the dS blocks the query-stationary dF_q kernel reads.  The
// element mask inside a block is the reference's (bucket relation, k <= q).
// The k = q - 1 term, when the buckets are not near, lies outside every
// window; each query adds it on its own (forward: one more online-softmax
// step; backward: the dK/dV kernel forms its dS for the key q - 1 and hands it
// to the dF_q kernel through one float per position).
//
// Sorted arrays per (b,h), T16 = 16 * ceil(T / 16) rows:
//   perm  [T16] position of sorted index j (-1 past T)
//   bsort [T16] bucket of sorted index j
//   cinfo [T16/16] int4 per 16-row chunk: bucket set, 0, min and max position
//   bstart[16]  first sorted index of each bucket (entries 0..8)
//   feat  [T16][32] features; lse, delta [T16] (backward)
// (the value and dO rows are read in place, through perm, by the kernels)
// dS of the sparse backward: [b*h][key tile of 64 sorted keys][T16 sorted
// queries][64], only the executed blocks written.
#include "wha_launch.hpp"

namespace wha {

namespace {
constexpr int kFP = kWaveFeatures;
constexpr int kLDF = kFP + 4;
constexpr int kNoPos = 0x7fffffff;

__device__ __forceinline__ int4 empty_chunk() { return make_int4(0, 0, kNoPos, -1); }

// Buckets within one of a bucket in the 8-bit set m.
__device__ __forceinline__ int near_set(int m) {
  return (m | (m << 1) | (m >> 1) | (m << 7) | (m >> 7)) & 0xff;
}

// Whether the 16 x 16 block (query chunk qc, key chunk kc) can hold an admitted pair.
__device__ __forceinline__ bool block_live(const int4& qc, const int4& kc) {
  return (near_set(qc.x) & kc.x) != 0 && kc.z <= qc.w;
}

// Chunks [c0, c0 + n) mod NC that hold every sorted index whose bucket is
// within one of a bucket in [bf, bl] (the buckets of one 64-row tile: sorted,
// so bf <= bl).
__device__ __forceinline__ void bucket_window(const int* bst, int bf, int bl, int NC, int& c0, int& n) {
  if (bl - bf >= 5) {
    c0 = 0;
    n = NC;
    return;
  }
  const int lo = (bf + 7) & 7, hi = (bl + 1) & 7;
  const int cs = bst[lo] >> 4, ce = (bst[hi + 1] + 15) >> 4;
  const int len = lo <= hi ? ce - cs : NC - cs + ce;
  if (len >= NC) {
    c0 = 0;
    n = NC;
    return;
  }
  c0 = cs < NC ? cs : 0;
  n = len > 0 ? len : 0;
}

// Chunk id of window offset o (o < n + 3 <= NC + 3): at most two wraps.
__device__ __forceinline__ int window_chunk(int c0, int o, int NC) {
  int c = c0 + o;
  if (c >= NC) c -= NC;
  if (c >= NC) c -= NC;
  return c;
}

// One of four values by a small index (a select chain, not a dynamically
// indexed array, which would go to scratch memory).
__device__ __forceinline__ int sel4(const int (&a)[4], int m) {
  return m == 0 ? a[0] : m == 1 ? a[1] : m == 2 ? a[2] : a[3];
}

// A stage of 64 sorted rows: the window chunks c0 + 4 kt .. + 3 (wave-uniform
// values): the first sorted row of each chunk and its description (empty for
// chunks past the window).
struct StageInfo {
  int row0[4];
  int4 ci[4];
};
__device__ __forceinline__ void stage_info(const int4* __restrict__ CIh, int c0, int kt, int n_ch, int NC,
                                           StageInfo& st) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int c = window_chunk(c0, 4 * kt + m, NC);
    st.row0[m] = 16 * c;
    st.ci[m] = 4 * kt + m < n_ch ? CIh[c] : empty_chunk();
  }
}

// 64 rows of W floats (W % 4 == 0) of a sorted [T16][W] array: row r of the
// stage is sorted row row0[r / 16] + r % 16 (zeros at and past T), staged
// through registers into an LDS tile of pitch LD by NT threads.
template <int W, int LD, int NT = 256>
struct ChunkRows {
  static constexpr int Q = W / 4;
  static constexpr int PER = (64 * Q + NT - 1) / NT;
  float4 r[PER];
  __device__ __forceinline__ void load(const float* __restrict__ base, const int (&row0)[4], int T, int tid) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + NT * p;
      const int row = idx / Q, q = idx % Q;
      const int j = sel4(row0, row >> 4) + (row & 15);
      r[p] = (idx < 64 * Q && j < T) ? *reinterpret_cast<const float4*>(base + (unsigned)(j * W + 4 * q))
                                     : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + NT * p;
      if (idx < 64 * Q) *reinterpret_cast<float4*>(lds + (idx / Q) * LD + 4 * (idx % Q)) = r[p];
    }
  }
};

// 64 rows of DP floats gathered from a head slice of a [B][T][E] tensor in
// sorted order: row r of the stage is position pos of sorted row
// row0[r / 16] + r % 16, zero padded past D and for rows at and past T.  The
// positions are fetched one stage ahead (load_pos), so the row loads of a
// stage do not wait on them.
template <int DP, int LD, bool VEC, int NT = 256>
struct GatherRows {
  static constexpr int Q = DP / 4;
  static constexpr int PER = (64 * Q + NT - 1) / NT;
  float4 r[PER];
  int pos[PER];
  __device__ __forceinline__ void load_pos(const int* __restrict__ PSh, const int (&row0)[4], int T, int tid) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + NT * p;
      const int row = idx / Q;
      const int j = sel4(row0, row >> 4) + (row & 15);
      pos[p] = (idx < 64 * Q && j < T) ? PSh[j] : -1;
    }
  }
  __device__ __forceinline__ void load(const float* __restrict__ Xh, int64_t st, int D, int tid) {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int q = (tid + NT * p) % Q;
      float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
      if (pos[p] >= 0) {
        const float* src = Xh + (int64_t)pos[p] * st + 4 * q;
        if (VEC) {
          if (4 * q < D) v = *reinterpret_cast<const float4*>(src);
        } else {
          if (4 * q + 0 < D) v.x = src[0];
          if (4 * q + 1 < D) v.y = src[1];
          if (4 * q + 2 < D) v.z = src[2];
          if (4 * q + 3 < D) v.w = src[3];
        }
      }
      r[p] = v;
    }
  }
  __device__ __forceinline__ void store(float* lds, int tid) const {
#pragma unroll
    for (int p = 0; p < PER; ++p) {
      const int idx = tid + NT * p;
      if (idx < 64 * Q) *reinterpret_cast<float4*>(lds + (idx / Q) * LD + 4 * (idx % Q)) = r[p];
    }
  }
};
}  // namespace

// ------------------------------------------------------------ sort and gather

// Stable counting sort of one (b,h)'s positions by bucket.  Block = one (b,h),
// kSortThreads threads; positions are placed kSortThreads at a time: rank
// within the wave from ballots, offsets of earlier waves and earlier passes
// from LDS counters.
constexpr int kSortThreads = 1024;
constexpr int kSortWaves = kSortThreads / 64;
__global__ __launch_bounds__(kSortThreads) void wave_sort_kernel(const int* __restrict__ BK, int* __restrict__ perm,
                                                                 int* __restrict__ bsort, int* __restrict__ bstart,
                                                                 int T, int T16) {
  __shared__ int cnt[8], base[8], wc[kSortWaves][8];
  const int bh = blockIdx.x;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int* bk = BK + (int64_t)bh * T;
  int* pm = perm + (int64_t)bh * T16;
  int* bs = bsort + (int64_t)bh * T16;
  if (tid < 8) cnt[tid] = 0;
  __syncthreads();
  for (int p = tid; p < T; p += kSortThreads) atomicAdd(&cnt[bk[p] & 7], 1);
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int v = 0; v < 8; ++v) {
      base[v] = acc;
      bstart[bh * 16 + v] = acc;
      acc += cnt[v];
    }
    bstart[bh * 16 + 8] = acc;
  }
  __syncthreads();
  const unsigned long long below = (1ull << lane) - 1ull;
  for (int p0 = 0; p0 < T; p0 += kSortThreads) {
    const int p = p0 + tid;
    const int b = p < T ? (bk[p] & 7) : 8;
    int rank = 0;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      const unsigned long long m = __ballot(b == v);
      if (b == v) rank = __popcll(m & below);
      if (lane == 0) wc[wave][v] = __popcll(m);
    }
    __syncthreads();
    if (b < 8) {
      int off = base[b] + rank;
      for (int w = 0; w < wave; ++w) off += wc[w][b];
      pm[off] = p;
      bs[off] = b;
    }
    __syncthreads();
    if (tid < 8) {
      int add = 0;
      for (int w = 0; w < kSortWaves; ++w) add += wc[w][tid];
      base[tid] += add;
    }
    __syncthreads();
  }
  for (int j = T + tid; j < T16; j += kSortThreads) {
    pm[j] = -1;
    bs[j] = 0;
  }
}

// Gathers into sorted order (block = 64 sorted rows of one (b,h)): the
// feature rows; LSE and Delta, when given; and the descriptions of the
// block's four chunks.  (Value and dO rows are gathered by the attention
// kernels themselves.)
__global__ __launch_bounds__(256) void wave_gather_kernel(const int* __restrict__ perm,
                                                          const int* __restrict__ bsort,
                                                          const float* __restrict__ F,
                                                          const float* __restrict__ lse,
                                                          const float* __restrict__ delta, float* __restrict__ FS,
                                                          float* __restrict__ LS, float* __restrict__ DLS,
                                                          int4* __restrict__ CI, View Lv) {
  const int T = Lv.T, BH = Lv.B * Lv.H;
  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  const int bh = blockIdx.x % BH, rg = (int)(blockIdx.x / BH);
  const int tid = threadIdx.x;
  const int j0 = 64 * rg;
  const int* pm = perm + (int64_t)bh * T16;
  const float* Fh = F + (int64_t)bh * T * kFP;
  // features: 64 rows x 8 quads
  for (int e = tid; e < 64 * (kFP / 4); e += 256) {
    const int j = j0 + e / (kFP / 4), q = e % (kFP / 4);
    if (j >= T16) continue;
    const int pos = pm[j];
    const float4 v = pos >= 0 ? *reinterpret_cast<const float4*>(Fh + (int64_t)pos * kFP + 4 * q)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    *reinterpret_cast<float4*>(FS + ((int64_t)bh * T16 + j) * kFP + 4 * q) = v;
  }
  if (lse != nullptr && tid < 64 && j0 + tid < T16) {
    const int j = j0 + tid;
    const int pos = pm[j];
    LS[(int64_t)bh * T16 + j] = pos >= 0 ? lse[(int64_t)bh * T + pos] : 0.f;
    DLS[(int64_t)bh * T16 + j] = pos >= 0 ? delta[(int64_t)bh * T + pos] : 0.f;
  }
  if (tid < 4) {
    const int c = 4 * rg + tid;
    if (c < NC) {
      const int* bs = bsort + (int64_t)bh * T16;
      int set = 0, lo = kNoPos, hi = -1;
      for (int j = 16 * c; j < min(16 * c + 16, T); ++j) {
        set |= 1 << bs[j];
        lo = min(lo, pm[j]);
        hi = max(hi, pm[j]);
      }
      CI[(int64_t)bh * NC + c] = make_int4(set, 0, lo, hi);
    }
  }
}

// ------------------------------------------------------------ forward

// Query-stationary forward over sorted queries.  Block = 64 sorted queries of
// one (b,h) (4 waves x 16, one query per lane), keys = the tile's bucket
// window, 64 keys (four chunks) per LDS stage; S^T = F_k F_q^T (keys on MFMA
// rows) and O^T += V^T P^T as in wave_fwd_kernel, per 16-key chunk only where
// block_live().  The k = q - 1 term (buckets not near) is one more online
// softmax step per lane before the output is scattered to the query's position.
template <int DP, bool VEC, int NW>
__global__ __launch_bounds__(NW * 64) void wave_sfwd_kernel(const float* __restrict__ FS, const int* __restrict__ PS,
                                                        const int* __restrict__ BSs,
                                                        const int4* __restrict__ CI, const int* __restrict__ BST,
                                                        const float* __restrict__ F, const int* __restrict__ BK,
                                                        const float* __restrict__ V, float* __restrict__ O,
                                                        float* __restrict__ LSE, View Lv, float cs) {
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int NDT = DP / 16, DG = DP / 4, FG = kFP / 4;
  __shared__ __align__(16) float Fs[64 * kLDF];
  __shared__ __align__(16) float Vs[64 * LD];
  __shared__ __align__(16) int Bs[64];  // bucket bit 1 << bucket of each key (0 past T)
  __shared__ __align__(16) int Ps[64];  // position of each key

  constexpr int QT = 16 * NW;  // sorted queries per block
  const int T = Lv.T, BH = Lv.B * Lv.H;
  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  const int n_qt = (T + QT - 1) / QT;
  const int bh = blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* FSh = FS + (int64_t)bh * T16 * kFP;
  const int* PSh = PS + (int64_t)bh * T16;
  const int* BSh = BSs + (int64_t)bh * T16;
  const int4* CIh = CI + (int64_t)bh * NC;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int qc = NW * qt + wave;
  const int qrow = 16 * qc + lq;
  const bool qok = qrow < T;

  float qf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      // unconditional loads (row 0 stands in past T), so they issue together
      qf[e] = FSh[(int64_t)(qok ? qrow : 0) * kFP + f] * (f < 2 ? kLog2e : w_cs);
      qf[e] = qok ? qf[e] : 0.f;
    }
  }
  const int qb = qok ? BSh[qrow] : 0;
  const int qpos = qok ? PSh[qrow] : -1;
  // bucket of the previous position, for the k = q - 1 term (fetched now, used last)
  const int pb = qok && qpos >= 1 ? Bh[qpos - 1] : 0;
  const int nq = qok ? near_set(1 << qb) : 0;  // buckets this query admits
  const int4 ci = qc < NC ? CIh[qc] : empty_chunk();

  int c0, n_ch;
  bucket_window(BST + bh * 16, BSh[QT * qt], BSh[min(QT * qt + QT - 1, T - 1)], NC, c0, n_ch);
  const int n_kt = (n_ch + 3) >> 2;

  // nxt: the stage whose rows load() fetches (its value-row positions already
  // in vs.pos); nxt2: the stage after it, whose positions load() requests
  StageInfo nxt, nxt2;
  ChunkRows<kFP, kLDF, NW * 64> fs;
  GatherRows<DP, LD, VEC, NW * 64> vs;
  int kb_r = 0, kp_r = -1;  // raw bucket: its bit is formed when stored, not beside the load
  auto load = [&](int kt) {
    fs.load(FSh, nxt.row0, T, tid);
    vs.load(V + vbase, Lv.st, Lv.D, tid);
    if (tid < 64) {
      const int j = sel4(nxt.row0, tid >> 4) + (tid & 15);
      kb_r = j < T ? BSh[j] : 0;
      kp_r = j < T ? PSh[j] : -1;
    }
    if (kt + 1 < n_kt) {
      stage_info(CIh, c0, kt + 1, n_ch, NC, nxt2);
      vs.load_pos(PSh, nxt2.row0, T, tid);
    }
  };
  if (n_kt > 0) {
    stage_info(CIh, c0, 0, n_ch, NC, nxt);
    vs.load_pos(PSh, nxt.row0, T, tid);
    load(0);
  }

  float m_i = -1e30f, l_i = 0.f;
  floatx4 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < n_kt; ++kt) {
    // live chunks of this stage for this wave (wave-uniform)
    int on = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) on |= block_live(ci, nxt.ci[m]) ? 1 << m : 0;
    __syncthreads();
    fs.store(Fs, tid);
    vs.store(Vs, tid);
    if (tid < 64) {
      Bs[tid] = kp_r >= 0 ? 1 << kb_r : 0;
      Ps[tid] = kp_r;
    }
    __syncthreads();
    if (kt + 1 < n_kt) {
      nxt = nxt2;
      load(kt + 1);
    }
    if (on == 0) continue;

    floatx4 s[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      s[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (on & (1 << mt)) {
#pragma unroll
        for (int j = 0; j < FG / 4; ++j) {
          const float4 a = *reinterpret_cast<const float4*>(&Fs[(16 * mt + lq) * kLDF + g * FG + 4 * j]);
          s[mt] = mfma4(a.x, qf[4 * j + 0], s[mt]);
          s[mt] = mfma4(a.y, qf[4 * j + 1], s[mt]);
          s[mt] = mfma4(a.z, qf[4 * j + 2], s[mt]);
          s[mt] = mfma4(a.w, qf[4 * j + 3], s[mt]);
        }
      }
    }

    // lane element (mt, i): key 16mt+4g+i of the stage, query lq
    float mx = -INFINITY;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (on & (1 << mt)) {
        const int4 kb4 = *reinterpret_cast<const int4*>(&Bs[16 * mt + 4 * g]);
        const int4 kp4 = *reinterpret_cast<const int4*>(&Ps[16 * mt + 4 * g]);
        const int kbv[4] = {kb4.x, kb4.y, kb4.z, kb4.w};
        const int kpv[4] = {kp4.x, kp4.y, kp4.z, kp4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool valid = (kpv[i] <= qpos) & ((nq & kbv[i]) != 0);
          const float x = valid ? s[mt][i] : -INFINITY;
          s[mt][i] = x;
          mx = fmaxf(mx, x);
        }
      }
    }
    mx = pair_max32(pair_max16(mx));
    const float m_new = fmaxf(m_i, mx);
    const float alpha = fast_exp2(m_i - m_new);
    float rs = 0.f;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (on & (1 << mt)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p = fast_exp2(s[mt][i] - m_new);
          s[mt][i] = p;
          rs += p;
        }
      }
    }
    l_i = l_i * alpha + rs;
    m_i = m_new;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (on & (1 << mt)) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float va[NDT];
          lds_read_seg<DP, NDT>(Vs, 16 * mt + 4 * g + i, lq, va);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma4(va[dt], s[mt][i], oacc[dt]);
        }
      }
    }
  }

  // the previous position when its bucket is not near (outside every window)
  const int pp = qpos - 1;
  const bool extra = qok && pp >= 0 && !wave_bucket_near(pb, qb);
  float part = 0.f;
  if (extra) {
#pragma unroll
    for (int e = 0; e < FG; ++e) part += qf[e] * Fh[(int64_t)pp * kFP + g * FG + e];
  }
  const float sx = pair_sum32(pair_sum16(part));
  if (extra) {
    const float m_new = fmaxf(m_i, sx);
    const float alpha = fast_exp2(m_i - m_new);
    const float px = fast_exp2(sx - m_new);
    l_i = l_i * alpha + (g == 0 ? px : 0.f);
    m_i = m_new;
    float vp[DG];
    load_row_frag<DP, VEC>(V + vbase, pp, T, Lv.D, Lv.st, g, 1.f, vp);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] * alpha + px * vp[NDT * i + dt];
    }
  }

  const float l_sum = pair_sum32(pair_sum16(l_i));
  const float inv = qok ? 1.f / l_sum : 0.f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] * inv;
  }
  store_row_frag<DP, VEC>(O + vbase, qok ? qpos : T, T, Lv.D, Lv.st, g, oacc, 1.f);
  if (LSE != nullptr && g == 0 && qok) LSE[(int64_t)bh * T + qpos] = (m_i + log2f(l_sum)) * kLn2;
}

// The same forward with one wave per workgroup (16 sorted queries), no LDS
// staging and no workgroup barrier.  The wave lists the live key chunks of its
// own query chunk (the bucket window of its own buckets, block_live per
// 16-key chunk) in LDS, then walks them with every operand loaded straight
// into the MFMA operand registers, NS - 1 chunks ahead of the one it computes
// (NS register sets; the key positions, which address the value rows, one
// step before the rows; NS = 2 at four waves per SIMD measured ahead of
// NS = 3 at three and NS = 4 at two).  A wave's time is then the sum of its own live
// chunks rather than, per 64-key stage, the most any wave of a block had, and
// a CU holds as many chunks in flight as its waves have registers.  Lane
// (lq, g) loads features 8g .. 8g+7 of key row lq (the S = F_k F_q^T A
// operand: two 16-byte loads; the 16 rows of a chunk are contiguous in sorted
// order) and, for keys 4g + i, value quad lq of the key's row (the O += V^T
// P^T A operand, gathered through the permutation), with the positions and
// buckets of keys 4g .. 4g+3 for the mask; buffer loads, so a chunk's offset
// is one scalar.  Every step issues the same loads (past the last live chunk,
// repeats of it that are never used), so the compiler's count of loads in
// flight stays exact.  Chunks the mask admits whole (flagged in the list) skip
// the element mask, and the running max moves only when a query's maximum
// passes it by more than kSparseLazy.  D padded to 64, 16-byte aligned value
// rows (vec).
#ifndef WHA_SFWD_NS
#define WHA_SFWD_NS 2
#endif
constexpr float kSparseLazy = 8.f;  // log2 units
template <bool PADQ, int NS = WHA_SFWD_NS>
__global__ __launch_bounds__(64) __attribute__((amdgpu_waves_per_eu(NS <= 2 ? 4 : NS == 3 ? 3 : 2))) void wave_sfwd_reg_kernel(
    const float* __restrict__ FS, const int* __restrict__ PS, const int* __restrict__ BSs,
    const int4* __restrict__ CI, const int* __restrict__ BST, const float* __restrict__ F,
    const int* __restrict__ BK, const float* __restrict__ V, float* __restrict__ O, float* __restrict__ LSE, View Lv,
    float cs) {
  constexpr int DP = 64;
  constexpr int NDT = DP / 16, FG = kFP / 4;
  static_assert(FG == 8, "32 features: two 16-byte loads per lane");
  extern __shared__ int live_list[];  // NC entries

  const int T = Lv.T, BH = Lv.B * Lv.H;
  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  // workgroup -> (head, query chunk).  Workgroups are dealt to the 8 XCDs in
  // turn; with BH % 8 == 0 every chunk of a head lands on one XCD, whose L2
  // then serves the head's gathered rows to all of them.
  const int wg = (int)blockIdx.x;
  int bh, qc;
  if (BH % 8 == 0) {
    bh = (wg & 7) + 8 * ((wg >> 3) / NC);
    qc = (wg >> 3) % NC;
  } else {
    bh = wg % BH;
    qc = wg / BH;
  }
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* FSh = FS + (int64_t)bh * T16 * kFP;
  const int* PSh = PS + (int64_t)bh * T16;
  const int* BSh = BSs + (int64_t)bh * T16;
  const int4* CIh = CI + (int64_t)bh * NC;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;

  const int lane = (int)threadIdx.x;
  const int lq = lane & 15, g = lane >> 4;
  const int qrow = 16 * qc + lq;
  const bool qok = qrow < T;

  float qf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      qf[e] = FSh[(int64_t)(qok ? qrow : 0) * kFP + f] * (f < 2 ? kLog2e : w_cs);
      qf[e] = qok ? qf[e] : 0.f;
    }
  }
  const int qb = qok ? BSh[qrow] : 0;
  const int qpos = qok ? PSh[qrow] : -1;
  const int pb = qok && qpos >= 1 ? Bh[qpos - 1] : 0;
  const int nq = qok ? near_set(1 << qb) : 0;
  const int4 ci = CIh[qc];

  int c0, n_ch;
  bucket_window(BST + bh * 16, BSh[16 * qc], BSh[min(16 * qc + 15, T - 1)], NC, c0, n_ch);

  // buckets every query of the chunk admits (the chunk's bucket set ci.x)
  int nq_all = 0xff;
#pragma unroll
  for (int v = 0; v < 8; ++v) nq_all &= ((ci.x >> v) & 1) ? near_set(1 << v) : 0xff;
  // the live chunks of the window, in window order, with bit 31 set on chunks
  // every pair of which the mask admits: all 16 keys before T, their buckets
  // admitted by every query bucket of the chunk, and no key after its first
  // query (those skip the per-element mask)
  int n_live = 0;
  for (int o0 = 0; o0 < n_ch; o0 += 64) {
    const int o = o0 + lane;
    const int c = window_chunk(c0, o < n_ch ? o : 0, NC);
    const int4 kc = CIh[c];
    const bool on = o < n_ch && block_live(ci, kc);
    const bool full = (kc.x & ~nq_all) == 0 && kc.w <= ci.z && 16 * c + 16 <= T;
    const uint64_t m = __ballot(on);
    if (on)
      live_list[n_live + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] =
          c | (full ? (int)0x80000000u : 0);
    n_live += __builtin_popcountll(m);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the list is in LDS
  __builtin_amdgcn_wave_barrier();

  // buffers over this head's sorted features, positions and buckets (a
  // chunk's rows at a uniform offset) and its value rows (this lane's quad of
  // row r at r * st + 4 lq floats; a quad past D reads quad 0 instead: it only
  // feeds output columns that are never stored)
  const __amdgpu_buffer_rsrc_t rF = buffer_rsrc(FSh, (uint32_t)T16 * kFP * 4u);
  const __amdgpu_buffer_rsrc_t rP = buffer_rsrc(PSh, (uint32_t)T16 * 4u);
  const __amdgpu_buffer_rsrc_t rB = buffer_rsrc(BSh, (uint32_t)T16 * 4u);
  const uint32_t st4 = 4u * (uint32_t)Lv.st;  // < 2^24, and the slice < 4 GiB (checked on the host)
  const __amdgpu_buffer_rsrc_t rV =
      buffer_rsrc(V + vbase, (uint32_t)((uint64_t)(T - 1) * st4 + 4u * (uint32_t)Lv.D));
  const int vq = (PADQ && 4 * lq >= Lv.D) ? 0 : 16 * lq;
  const int foff = (lq * kFP + 8 * g) * 4, koff = 16 * g;

  // the k-th live chunk entry (past the end: the last one again, never computed)
  auto chunk_at = [&](int k) { return __builtin_amdgcn_readfirstlane(live_list[min(k, n_live - 1)]); };
  struct Set {
    float4 f0, f1;  // features 8g .. 8g+7 of key row lq
    float4 v[4];    // value quad lq of keys 4g + i
    int4 p, b;      // positions and buckets of keys 4g .. 4g+3
    int full;       // the list entry: negative when no element mask is needed
  };
  auto ld_int4 = [&](__amdgpu_buffer_rsrc_t r, int voff, int soff) {
    typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
    const uintx4 v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0);
    return make_int4((int)v[0], (int)v[1], (int)v[2], (int)v[3]);
  };
  auto load_pos = [&](int e) { return ld_int4(rP, koff, 64 * (e & 0x7fffffff)); };
  auto load_set = [&](int e, const int4& p, Set& d) {
    const int c = e & 0x7fffffff;
    d.f0 = buffer_load_quad(rF, foff, c * (16 * kFP * 4));
    d.f1 = buffer_load_quad(rF, foff + 16, c * (16 * kFP * 4));
    // keys past T (position -1) read position 0 and are masked
    const int pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int i = 0; i < 4; ++i)
      d.v[i] = buffer_load_quad(rV, (int)(__umul24((uint32_t)max(pv[i], 0), st4) + (uint32_t)vq), 0);
    d.b = ld_int4(rB, koff, 64 * c);
    d.p = p;
    d.full = e;
  };

  float m_i = -1e30f, l_i = 0.f;
  floatx4 oacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) oacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](const Set& d) {
    // S^T[key 4g + i][query lq] of the chunk, log2 units
    floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f};
    s = mfma4(d.f0.x, qf[0], s);
    s = mfma4(d.f0.y, qf[1], s);
    s = mfma4(d.f0.z, qf[2], s);
    s = mfma4(d.f0.w, qf[3], s);
    s = mfma4(d.f1.x, qf[4], s);
    s = mfma4(d.f1.y, qf[5], s);
    s = mfma4(d.f1.z, qf[6], s);
    s = mfma4(d.f1.w, qf[7], s);
    if (d.full >= 0) {
      const int kp[4] = {d.p.x, d.p.y, d.p.z, d.p.w};
      const int kb[4] = {d.b.x, d.b.y, d.b.z, d.b.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const bool valid = (kp[i] >= 0) & (kp[i] <= qpos) & (((nq >> kb[i]) & 1) != 0);
        s[i] = valid ? s[i] : -INFINITY;
      }
    }
    const float mx = vmax3(vmax3(s[0], s[1], s[2]), s[3], s[3]);
    // the running max moves only when some query's maximum passes it by more
    // than kSparseLazy (or it is still the initial floor): the probabilities
    // then stay below 2^kSparseLazy, and the result (O and LSE) does not depend
    // on which maximum was subtracted
    if (__builtin_amdgcn_ballot_w64(mx > m_i + kSparseLazy) != 0) {
      // its new maximum over the four lane groups
      const float m_new = fmaxf(m_i, pair_max32(pair_max16(mx)));
      const float alpha = fast_exp2(m_i - m_new);
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] *= alpha;
      m_i = m_new;
    }
    float rs = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      s[i] = fast_exp2(s[i] - m_i);
      rs += s[i];
    }
    l_i += rs;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float va[4] = {d.v[i].x, d.v[i].y, d.v[i].z, d.v[i].w};
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[dt] = mfma4(va[dt], s[i], oacc[dt]);
    }
  };

  if (n_live > 0) {
    // chunk j: positions in pos set j % NS (requested at step j - NS), operands
    // in set j % NS (requested at step j - NS + 1, from those positions),
    // computed at step j; chunk ids read from the list one step before use
    Set sets[NS];
    int4 ps[NS];
    auto list_at = [&](int k) { return live_list[min(k, n_live - 1)]; };
#pragma unroll
    for (int j = 0; j < NS; ++j) ps[j] = load_pos(chunk_at(j));
    WHA_FENCE();
#pragma unroll
    for (int j = 0; j < NS - 1; ++j) {
      load_set(chunk_at(j), ps[j], sets[j]);
      WHA_FENCE();
    }
    int id_set = chunk_at(NS - 1);  // the chunk whose operands the next step requests
    int id_v = list_at(NS);         // the chunk whose positions it requests (a lane value)
    // whole rounds of NS steps: a step past the last chunk only loads; the
    // skipped computations issue no loads, so every path through a round
    // issues the same ones
    int k = 0;
    do {
#pragma unroll
      for (int u = 0; u < NS; ++u) {
        const int id_pos = __builtin_amdgcn_readfirstlane(id_v);
        id_v = list_at(k + u + NS + 1);
        WHA_FENCE();
        ps[u] = load_pos(id_pos);
        WHA_FENCE();
        load_set(id_set, ps[(u + NS - 1) % NS], sets[(u + NS - 1) % NS]);
        WHA_FENCE();
        id_set = id_pos;
        if (k + u < n_live) compute(sets[u]);
      }
      k += NS;
    } while (k < n_live);
    wait_vmem();  // the loads past the end land before the wave ends
  }

  // the previous position when its bucket is not near (outside every window)
  const int pp = qpos - 1;
  const bool extra = qok && pp >= 0 && !wave_bucket_near(pb, qb);
  float part = 0.f;
  if (extra) {
#pragma unroll
    for (int e = 0; e < FG; ++e) part += qf[e] * Fh[(int64_t)pp * kFP + g * FG + e];
  }
  const float sx = pair_sum32(pair_sum16(part));
  if (extra) {
    const float m_new = fmaxf(m_i, sx);
    const float alpha = fast_exp2(m_i - m_new);
    const float px = fast_exp2(sx - m_new);
    l_i = l_i * alpha + (g == 0 ? px : 0.f);
    m_i = m_new;
    float vp[DP / 4];
    load_row_frag<DP, true>(V + vbase, pp, T, Lv.D, Lv.st, g, 1.f, vp);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] * alpha + px * vp[NDT * i + dt];
    }
  }

  const float l_sum = pair_sum32(pair_sum16(l_i));
  const float inv = qok ? 1.f / l_sum : 0.f;
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
    for (int i = 0; i < 4; ++i) oacc[dt][i] = oacc[dt][i] * inv;
  }
  store_row_frag<DP, true>(O + vbase, qok ? qpos : T, T, Lv.D, Lv.st, g, oacc, 1.f);
  if (LSE != nullptr && g == 0 && qok) LSE[(int64_t)bh * T + qpos] = (m_i + log2f(l_sum)) * kLn2;
}

// ------------------------------------------------------------ backward

// Key-stationary backward over sorted keys.  Block = 64 sorted keys of one
// (b,h) (4 waves x 16, one key per lane), queries = the tile's bucket window,
// 64 per LDS stage; per live 16 x 16 block S and dP (queries on MFMA rows),
// P = exp2(S - LSE log2 e), dS = P (dP - Delta), dV^T += dO^T P, dF_k^T +=
// F_q^T dS, and the dS block stored for the dF_q kernel.  Then the k = q - 1
// term of the query at position k + 1 (buckets not near): its P, dS added to
// this key's dV and dF_k, and its dS written to dsp[position k + 1] (0 where
// the term does not apply).  dV, dF_k are scattered to the key's position.
template <int DP, bool VEC>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(DP == 128 ? 2 : 3))) void wave_sdkv_kernel(
    const float* __restrict__ FS, const float* __restrict__ LS, const float* __restrict__ DLS,
    const int* __restrict__ PS, const int* __restrict__ BSs, const int4* __restrict__ CI,
    const int* __restrict__ BST, const float* __restrict__ F, const int* __restrict__ BK,
    const float* __restrict__ V, const float* __restrict__ dO,
    const float* __restrict__ LSE, const float* __restrict__ Delta, float* __restrict__ dF, float* __restrict__ dV,
    float* __restrict__ DS, float* __restrict__ DSP, View Lv, float cs) {
  constexpr int LD = Lds<DP>::PITCH;
  constexpr int NDT = DP / 16, DG = DP / 4, FG = kFP / 4, NFT = kFP / 16;
  __shared__ __align__(16) float Fs[64 * kLDF];
  __shared__ __align__(16) float Os[64 * LD];
  __shared__ __align__(16) float lse_s[64];
  __shared__ __align__(16) float del_s[64];
  __shared__ __align__(16) int qb_s[64];  // bucket bit of each query (0 past T)
  __shared__ __align__(16) int qp_s[64];  // position of each query

  const int T = Lv.T, BH = Lv.B * Lv.H;
  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  const int n_kt_all = (T + 63) >> 6;
  const int bh = blockIdx.x % BH;
  const int kt = (int)(blockIdx.x / BH);
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* FSh = FS + (int64_t)bh * T16 * kFP;
  const float* LSh = LS + (int64_t)bh * T16;
  const float* DLh = DLS + (int64_t)bh * T16;
  const int* PSh = PS + (int64_t)bh * T16;
  const int* BSh = BSs + (int64_t)bh * T16;
  const int4* CIh = CI + (int64_t)bh * NC;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;
  const int64_t rbase = (int64_t)bh * T;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int kc = 4 * kt + wave;
  const int krow = 16 * kc + lq;
  const bool kok = krow < T;
  const int kpos = kok ? PSh[krow] : -1;
  const int kb = kok ? BSh[krow] : 0;
  const int nk = kok ? near_set(1 << kb) : 0;  // buckets of the queries this key meets
  const int4 ci = kc < NC ? CIh[kc] : empty_chunk();

  float kf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      // unconditional loads (row 0 stands in past T), so they issue together
      kf[e] = FSh[(int64_t)(kok ? krow : 0) * kFP + f] * (f < 2 ? kLog2e : w_cs);
      kf[e] = kok ? kf[e] : 0.f;
    }
  }
  float vf[DG];
  load_row_frag<DP, VEC>(V + vbase, kok && kpos >= 0 ? kpos : T, T, Lv.D, Lv.st, g, 1.f, vf);
  // bucket, LSE and Delta of the query at position kpos + 1, for the k = q - 1
  // term (fetched now, used last)
  const int qn = kpos + 1;
  const bool has_qn = kok && kpos >= 0 && qn < T;
  const int qn_b = has_qn ? Bh[qn] : 0;
  const float qn_lse = has_qn ? LSE[rbase + qn] : 0.f;
  const float qn_del = has_qn ? Delta[rbase + qn] : 0.f;

  floatx4 dfacc[NFT], dvacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NFT; ++dt) dfacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  int c0, n_ch;
  bucket_window(BST + bh * 16, BSh[64 * kt], BSh[min(64 * kt + 63, T - 1)], NC, c0, n_ch);
  const int n_qt = (n_ch + 3) >> 2;

  // nxt: the stage whose rows load() fetches (its dO-row positions already in
  // os.pos); nxt2: the stage after it, whose positions load() requests
  StageInfo nxt, nxt2;
  ChunkRows<kFP, kLDF> fs;
  GatherRows<DP, LD, VEC> os;
  float lse_r = 0.f, del_r = 0.f;
  int qb_r = 0, qp_r = -1;  // raw bucket: its bit is formed when stored, not beside the load
  auto load = [&](int qt) {
    fs.load(FSh, nxt.row0, T, tid);
    os.load(dO + vbase, Lv.st, Lv.D, tid);
    if (tid < 64) {
      const int j = sel4(nxt.row0, tid >> 4) + (tid & 15);
      const bool ok = j < T;
      lse_r = ok ? LSh[j] : 0.f;
      del_r = ok ? DLh[j] : 0.f;
      qb_r = ok ? BSh[j] : 0;
      qp_r = ok ? PSh[j] : -1;
    }
    if (qt + 1 < n_qt) {
      stage_info(CIh, c0, qt + 1, n_ch, NC, nxt2);
      os.load_pos(PSh, nxt2.row0, T, tid);
    }
  };
  if (n_qt > 0) {
    stage_info(CIh, c0, 0, n_ch, NC, nxt);
    os.load_pos(PSh, nxt.row0, T, tid);
    load(0);
  }

  // dS of this wave's 16 keys: column 16 * wave + lq of the key tile's block
  float* dsk = DS + (int64_t)(bh * n_kt_all + kt) * T16 * 64 + 16 * wave + lq;
  for (int qt = 0; qt < n_qt; ++qt) {
    // live query chunks of this stage for this wave's keys (wave-uniform), and their rows
    int on = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) on |= block_live(nxt.ci[m], ci) ? 1 << m : 0;
    int qrow0[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) qrow0[m] = nxt.row0[m];
    __syncthreads();
    fs.store(Fs, tid);
    os.store(Os, tid);
    if (tid < 64) {
      lse_s[tid] = lse_r * kLog2e;
      del_s[tid] = del_r;
      qb_s[tid] = qp_r >= 0 ? 1 << qb_r : 0;
      qp_s[tid] = qp_r;
    }
    __syncthreads();
    if (qt + 1 < n_qt) {
      nxt = nxt2;
      load(qt + 1);
    }
    if (on == 0) continue;

    floatx4 s[4], dp[4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      s[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      dp[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      if (on & (1 << mt)) {
#pragma unroll
        for (int j = 0; j < FG / 4; ++j) {
          const float4 a = *reinterpret_cast<const float4*>(&Fs[(16 * mt + lq) * kLDF + g * FG + 4 * j]);
          s[mt] = mfma4(a.x, kf[4 * j + 0], s[mt]);
          s[mt] = mfma4(a.y, kf[4 * j + 1], s[mt]);
          s[mt] = mfma4(a.z, kf[4 * j + 2], s[mt]);
          s[mt] = mfma4(a.w, kf[4 * j + 3], s[mt]);
        }
#pragma unroll
        for (int j = 0; j < DG / 4; ++j) {
          const float4 c = *reinterpret_cast<const float4*>(&Os[(16 * mt + lq) * LD + g * DG + 4 * j]);
          dp[mt] = mfma4(c.x, vf[4 * j + 0], dp[mt]);
          dp[mt] = mfma4(c.y, vf[4 * j + 1], dp[mt]);
          dp[mt] = mfma4(c.z, vf[4 * j + 2], dp[mt]);
          dp[mt] = mfma4(c.w, vf[4 * j + 3], dp[mt]);
        }
      }
    }

    // lane element (mt, i): query 16mt+4g+i of the stage, key krow
#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (on & (1 << mt)) {
        const float4 l4 = *reinterpret_cast<const float4*>(&lse_s[16 * mt + 4 * g]);
        const float4 d4 = *reinterpret_cast<const float4*>(&del_s[16 * mt + 4 * g]);
        const int4 b4 = *reinterpret_cast<const int4*>(&qb_s[16 * mt + 4 * g]);
        const int4 p4 = *reinterpret_cast<const int4*>(&qp_s[16 * mt + 4 * g]);
        const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
        const float dv4[4] = {d4.x, d4.y, d4.z, d4.w};
        const int bv[4] = {b4.x, b4.y, b4.z, b4.w};
        const int pv[4] = {p4.x, p4.y, p4.z, p4.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const bool valid = (pv[i] >= kpos) & ((nk & bv[i]) != 0);
          float p = fast_exp2(s[mt][i] - lv[i]);
          p = valid ? p : 0.f;
          s[mt][i] = p;
          dp[mt][i] = p * (dp[mt][i] - dv4[i]);
        }
        // rows of the stage's chunk mt: qrow0[mt] + 4g + i (all inside T16)
        float* dsq = dsk + (int64_t)(qrow0[mt] + 4 * g) * 64;
#pragma unroll
        for (int i = 0; i < 4; ++i) dsq[i * 64] = dp[mt][i];
      }
    }

#pragma unroll
    for (int mt = 0; mt < 4; ++mt) {
      if (on & (1 << mt)) {
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
  }

  // the query at position kpos + 1 when its bucket is not near this key's
  const bool extra = has_qn && !wave_bucket_near(kb, qn_b);
  float sp = 0.f, dpp = 0.f;
  float dof[DG];
  float fq[FG];
  if (extra) {
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      fq[e] = Fh[(int64_t)qn * kFP + g * FG + e];
      sp += kf[e] * fq[e];
    }
    load_row_frag<DP, VEC>(dO + vbase, qn, T, Lv.D, Lv.st, g, 1.f, dof);
#pragma unroll
    for (int e = 0; e < DG; ++e) dpp += vf[e] * dof[e];
  }
  sp = pair_sum32(pair_sum16(sp));
  dpp = pair_sum32(pair_sum16(dpp));
  float dsx = 0.f;
  if (extra) {
    const float p = fast_exp2(sp - qn_lse * kLog2e);
    dsx = p * (dpp - qn_del);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dvacc[dt][i] += p * dof[NDT * i + dt];
    }
#pragma unroll
    for (int dt = 0; dt < NFT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dfacc[dt][i] += dsx * fq[NFT * i + dt];
    }
  }
  if (has_qn && g == 0) DSP[rbase + qn] = dsx;

  const int out_row = kok && kpos >= 0 ? kpos : T;
  store_row_frag<kFP, true>(dF + rbase * kFP, out_row, T, kFP, kFP, g, dfacc, 1.f);
  store_row_frag<DP, VEC>(dV + vbase, out_row, T, Lv.D, Lv.st, g, dvacc, 1.f);
}

// The same backward with one wave per workgroup (16 sorted keys) and no
// workgroup barrier: the wave lists the live query chunks of its own key chunk
// (the bucket window of its own buckets, block_live) in LDS, with bit 31 set on
// chunks the mask admits whole, and walks them with two private LDS slots:
// while it computes one chunk, the next chunk's 16 feature rows (contiguous in
// sorted order; quad c of row r stored at c ^ (r & 7)) and 16 dO rows
// (gathered through the permutation, swizzled 64-wide rows, LDS row 4u + g
// holding query 4g + u so that a lane's four positions are one 16-byte load)
// arrive by global_load_lds, and this lane's LSE, Delta and buckets of queries
// 4g .. 4g+3 by buffer loads; the positions one step earlier, since they
// address the rows.  Per chunk as in wave_sdkv_kernel: S and dP with queries
// on MFMA rows, P = exp2(S - LSE log2 e), dS = P (dP - Delta), the dS block
// stored for the dF_q kernel, dV^T += dO^T P and dF_k^T += F_q^T dS.  D padded
// to 64, 16-byte aligned dO rows (vec).
template <bool PADQ>
__global__ __launch_bounds__(64) void wave_sdkv_dma_kernel(
    const float* __restrict__ FS, const float* __restrict__ LS, const float* __restrict__ DLS,
    const int* __restrict__ PS, const int* __restrict__ BSs, const int4* __restrict__ CI,
    const int* __restrict__ BST, const float* __restrict__ F, const int* __restrict__ BK,
    const float* __restrict__ V, const float* __restrict__ dO,
    const float* __restrict__ LSE, const float* __restrict__ Delta, float* __restrict__ dF, float* __restrict__ dV,
    float* __restrict__ DS, float* __restrict__ DSP, View Lv, float cs) {
  constexpr int DP = 64;
  constexpr int NDT = DP / 16, DG = DP / 4, FG = kFP / 4, NFT = kFP / 16, QPR = DP / 4;
  constexpr int NFD = 16 * (kFP / 4) / 64;  // feature DMA instructions per chunk
  constexpr int NOD = 16 * QPR / 64;        // dO DMA instructions per chunk
  static_assert(NFD == 2 && NOD == 4 && NFT == 2, "16-row chunks of 32 features and 64-wide dO rows");
  using LT = Lds<DP, true>;
  __shared__ __align__(16) float Fs0[16 * kFP], Fs1[16 * kFP];
  __shared__ __align__(16) float Os0[16 * DP], Os1[16 * DP];
  extern __shared__ int live_list[];  // NC entries

  const int T = Lv.T, BH = Lv.B * Lv.H;
  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  const int n_kt_all = (T + 63) >> 6;
  // workgroup -> (head, key chunk), a head's chunks on one XCD when BH % 8 == 0
  const int wg = (int)blockIdx.x;
  int bh, kc;
  if (BH % 8 == 0) {
    bh = (wg & 7) + 8 * ((wg >> 3) / NC);
    kc = (wg >> 3) % NC;
  } else {
    bh = wg % BH;
    kc = wg / BH;
  }
  const int b = bh / Lv.H, h = bh % Lv.H;
  const int64_t vbase = (int64_t)b * Lv.sb + (int64_t)h * Lv.sh;
  const float* FSh = FS + (int64_t)bh * T16 * kFP;
  const int* PSh = PS + (int64_t)bh * T16;
  const int* BSh = BSs + (int64_t)bh * T16;
  const int4* CIh = CI + (int64_t)bh * NC;
  const float* Fh = F + (int64_t)bh * T * kFP;
  const int* Bh = BK + (int64_t)bh * T;
  const int64_t rbase = (int64_t)bh * T;

  const int lane = (int)threadIdx.x;
  const int lq = lane & 15, g = lane >> 4;
  const int krow = 16 * kc + lq;
  const bool kok = krow < T;
  const int kpos = kok ? PSh[krow] : -1;
  const int kb = kok ? BSh[krow] : 0;
  const int nk = kok ? near_set(1 << kb) : 0;  // buckets of the queries this key meets
  const int4 ci = CIh[kc];

  float kf[FG];
  {
    const float w_cs = cs * kLog2e;
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      const int f = g * FG + e;
      kf[e] = FSh[(int64_t)(kok ? krow : 0) * kFP + f] * (f < 2 ? kLog2e : w_cs);
      kf[e] = kok ? kf[e] : 0.f;
    }
  }
  float vf[DG];
  load_row_frag<DP, true>(V + vbase, kok && kpos >= 0 ? kpos : T, T, Lv.D, Lv.st, g, 1.f, vf);
  const int qn = kpos + 1;
  const bool has_qn = kok && kpos >= 0 && qn < T;
  const int qn_b = has_qn ? Bh[qn] : 0;
  const float qn_lse = has_qn ? LSE[rbase + qn] : 0.f;
  const float qn_del = has_qn ? Delta[rbase + qn] : 0.f;

  floatx4 dfacc[NFT], dvacc[NDT];
#pragma unroll
  for (int dt = 0; dt < NFT; ++dt) dfacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  int c0, n_ch;
  bucket_window(BST + bh * 16, BSh[16 * kc], BSh[min(16 * kc + 15, T - 1)], NC, c0, n_ch);

  // query buckets every key of the chunk admits (the chunk's bucket set ci.x)
  int nk_all = 0xff;
#pragma unroll
  for (int v = 0; v < 8; ++v) nk_all &= ((ci.x >> v) & 1) ? near_set(1 << v) : 0xff;
  // live query chunks in window order; bit 31: the mask admits every pair
  // (16 queries before T, every query bucket admitted by every key bucket, no
  // query before the chunk's last key)
  int n_live = 0;
  for (int o0 = 0; o0 < n_ch; o0 += 64) {
    const int o = o0 + lane;
    const int c = window_chunk(c0, o < n_ch ? o : 0, NC);
    const int4 qi = CIh[c];
    const bool on = o < n_ch && block_live(qi, ci);
    const bool full = (qi.x & ~nk_all) == 0 && qi.z >= ci.w && 16 * c + 16 <= T;
    const uint64_t m = __ballot(on);
    if (on)
      live_list[n_live + __builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0))] =
          c | (full ? (int)0x80000000u : 0);
    n_live += __builtin_popcountll(m);
  }
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the list is in LDS
  __builtin_amdgcn_wave_barrier();

  // DMA sources: feature DMA u fills stored quad l & 7 of row 8u + (l >> 3);
  // dO DMA u stored quad l & 15 of LDS row 4u + g (query 4g + u); a quad past
  // D reads quad 0 instead (it feeds only dV columns that are never stored)
  uint32_t foff[NFD];
#pragma unroll
  for (int u = 0; u < NFD; ++u) {
    const int r = 8 * u + (lane >> 3);
    foff[u] = (uint32_t)(r * kFP + 4 * ((lane & 7) ^ (r & 7))) * 4u;
  }
  uint32_t oq[NOD];
#pragma unroll
  for (int u = 0; u < NOD; ++u) {
    const int c = LT::pq_inv(4 * u + g, lane & 15);
    oq[u] = (PADQ && 4 * c >= Lv.D) ? 0u : 16u * (uint32_t)c;
  }
  const char* Oh = reinterpret_cast<const char*>(dO + vbase);
  const char* Fb = reinterpret_cast<const char*>(FSh);
  const uint32_t st4 = 4u * (uint32_t)Lv.st;  // < 2^24, and the slice < 4 GiB (checked on the host)
  const __amdgpu_buffer_rsrc_t rP = buffer_rsrc(PSh, (uint32_t)T16 * 4u);
  const __amdgpu_buffer_rsrc_t rB = buffer_rsrc(BSh, (uint32_t)T16 * 4u);
  const __amdgpu_buffer_rsrc_t rL = buffer_rsrc(LS + (int64_t)bh * T16, (uint32_t)T16 * 4u);
  const __amdgpu_buffer_rsrc_t rD = buffer_rsrc(DLS + (int64_t)bh * T16, (uint32_t)T16 * 4u);
  const int koff = 16 * g;
  auto ld_int4 = [&](__amdgpu_buffer_rsrc_t r, int soff) {
    typedef unsigned uintx4 __attribute__((ext_vector_type(4)));
    const uintx4 v = __builtin_amdgcn_raw_buffer_load_b128(r, koff, soff, 0);
    return make_int4((int)v[0], (int)v[1], (int)v[2], (int)v[3]);
  };
  auto chunk_at = [&](int k) { return __builtin_amdgcn_readfirstlane(live_list[min(k, n_live - 1)]); };
  struct Q {
    int4 p, b;    // positions and buckets of queries 4g .. 4g+3
    float4 l, d;  // their LSE (log2 units after scaling) and Delta
    int e;        // list entry
  };
  // positions of chunk entry e (they address its dO rows)
  auto load_pos = [&](int e) { return ld_int4(rP, 64 * (e & 0x7fffffff)); };
  auto issue = [&](int e, const int4& p, float* Fd, float* Od, Q& q) {
    const int c = e & 0x7fffffff;
    const char* fsrc = Fb + (size_t)c * (16 * kFP * 4);
#pragma unroll
    for (int u = 0; u < NFD; ++u) dma_quad(reinterpret_cast<const float*>(fsrc + foff[u]), Fd + 256 * u);
    const int pv[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
    for (int u = 0; u < NOD; ++u)
      dma_quad(reinterpret_cast<const float*>(Oh + (__umul24((uint32_t)max(pv[u], 0), st4) + oq[u])), Od + 256 * u);
    // (the positions again for the mask: a copy of p, which the next step
    // reloads, would tie the two registers and wait for that load)
    q.p = ld_int4(rP, 64 * c);
    q.b = ld_int4(rB, 64 * c);
    q.l = buffer_load_quad(rL, koff, 64 * c);
    q.d = buffer_load_quad(rD, koff, 64 * c);
    q.e = e;
  };

  const int kt = kc >> 2;
  float* dsk = DS + (int64_t)(bh * n_kt_all + kt) * T16 * 64 + 16 * (kc & 3) + lq;
  auto compute = [&](const float* Fs, const float* Os, const Q& q) {
    const int c = q.e & 0x7fffffff;
    // lane element i: query 4g + i of the chunk, key lq
    floatx4 s = floatx4{0.f, 0.f, 0.f, 0.f}, dp = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < FG / 4; ++j) {
      const float4 a = *reinterpret_cast<const float4*>(&Fs[lq * kFP + 4 * ((2 * g + j) ^ (lq & 7))]);
      s = mfma4(a.x, kf[4 * j + 0], s);
      s = mfma4(a.y, kf[4 * j + 1], s);
      s = mfma4(a.z, kf[4 * j + 2], s);
      s = mfma4(a.w, kf[4 * j + 3], s);
    }
#pragma unroll
    for (int j = 0; j < DG / 4; ++j) {
      // dO row of query lq (LDS row tr16(lq)), quads 4g .. 4g+3
      const float4 a = lds_read_quad<DP, true>(Os, tr16(lq), 4 * g + j);
      dp = mfma4(a.x, vf[4 * j + 0], dp);
      dp = mfma4(a.y, vf[4 * j + 1], dp);
      dp = mfma4(a.z, vf[4 * j + 2], dp);
      dp = mfma4(a.w, vf[4 * j + 3], dp);
    }
    const float lv[4] = {q.l.x, q.l.y, q.l.z, q.l.w};
    const float dv4[4] = {q.d.x, q.d.y, q.d.z, q.d.w};
    const int pv[4] = {q.p.x, q.p.y, q.p.z, q.p.w};
    const int bv[4] = {q.b.x, q.b.y, q.b.z, q.b.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float p = fast_exp2(s[i] - lv[i] * kLog2e);
      if (q.e >= 0) {
        const bool valid = (pv[i] >= kpos) & (pv[i] >= 0) & (((nk >> bv[i]) & 1) != 0);
        p = valid ? p : 0.f;
      }
      s[i] = p;
      dp[i] = p * (dp[i] - dv4[i]);
    }
    float* dsq = dsk + (int64_t)(16 * c + 4 * g) * 64;
#pragma unroll
    for (int i = 0; i < 4; ++i) dsq[i * 64] = dp[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float oa[NDT];
      lds_read_seg<DP, NDT, true>(Os, 4 * i + g, lq, oa);
      // features 2lq, 2lq + 1 of query 4g + i
      const int r = 4 * g + i;
      const float2 fa = *reinterpret_cast<const float2*>(&Fs[r * kFP + 4 * ((lq >> 1) ^ (r & 7)) + 2 * (lq & 1)]);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) dvacc[dt] = mfma4(oa[dt], s[i], dvacc[dt]);
      dfacc[0] = mfma4(fa.x, dp[i], dfacc[0]);
      dfacc[1] = mfma4(fa.y, dp[i], dfacc[1]);
    }
  };

  if (n_live > 0) {
    Q q0, q1;
    const int e0 = chunk_at(0);
    const int4 p0 = load_pos(e0);
    wait_vmem();
    issue(e0, p0, Fs0, Os0, q0);
    // entries for slot 1 (eb, positions pb) and slot 0 (ea, pa), each written in
    // one half of the loop and read in the other (no register copies)
    int eb = chunk_at(1), ea;
    int4 pb = load_pos(eb), pa;
    // step on slot 0 (entry k), then slot 1 (entry k + 1); every step issues the
    // same loads (past the end, the last entry again, never computed)
    int k = 0;
    do {
      wait_vmem();  // slot 0 holds entry k; entry k + 1's positions are in
      issue(eb, pb, Fs1, Os1, q1);
      ea = chunk_at(k + 2);
      pa = load_pos(ea);
      compute(Fs0, Os0, q0);
      if (k + 1 >= n_live) break;
      wait_vmem();  // slot 1 holds entry k + 1; entry k + 2's positions are in
      issue(ea, pa, Fs0, Os0, q0);
      eb = chunk_at(k + 3);
      pb = load_pos(eb);
      compute(Fs1, Os1, q1);
      k += 2;
    } while (k < n_live);
    wait_vmem();  // the loads past the end land before the wave ends
  }

  // the query at position kpos + 1 when its bucket is not near this key's
  const bool extra = has_qn && !wave_bucket_near(kb, qn_b);
  float sp = 0.f, dpp = 0.f;
  float dof[DG];
  float fq[FG];
  if (extra) {
#pragma unroll
    for (int e = 0; e < FG; ++e) {
      fq[e] = Fh[(int64_t)qn * kFP + g * FG + e];
      sp += kf[e] * fq[e];
    }
    load_row_frag<DP, true>(dO + vbase, qn, T, Lv.D, Lv.st, g, 1.f, dof);
#pragma unroll
    for (int e = 0; e < DG; ++e) dpp += vf[e] * dof[e];
  }
  sp = pair_sum32(pair_sum16(sp));
  dpp = pair_sum32(pair_sum16(dpp));
  float dsx = 0.f;
  if (extra) {
    const float p = fast_exp2(sp - qn_lse * kLog2e);
    dsx = p * (dpp - qn_del);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dvacc[dt][i] += p * dof[NDT * i + dt];
    }
#pragma unroll
    for (int dt = 0; dt < NFT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) dfacc[dt][i] += dsx * fq[NFT * i + dt];
    }
  }
  if (has_qn && g == 0) DSP[rbase + qn] = dsx;

  const int out_row = kok && kpos >= 0 ? kpos : T;
  store_row_frag<kFP, true>(dF + rbase * kFP, out_row, T, kFP, kFP, g, dfacc, 1.f);
  store_row_frag<DP, true>(dV + vbase, out_row, T, Lv.D, Lv.st, g, dvacc, 1.f);
}

// dF_q = dS F_k over sorted queries.  Block = 64 sorted queries of one (b,h)
// (4 waves x 16), keys = the tile's bucket window, 64 key feature rows per LDS
// stage; a wave reads the dS block of (its chunk, key chunk) exactly when
// block_live() holds, the blocks the dK/dV kernel wrote; then the k = q - 1
// term from dsp, and the row is scattered to the query's position.
__global__ __launch_bounds__(256) void wave_sdq_kernel(const float* __restrict__ FS, const int* __restrict__ PS,
                                                       const int* __restrict__ BSs, const int4* __restrict__ CI,
                                                       const int* __restrict__ BST, const float* __restrict__ F,
                                                       const float* __restrict__ DS, const float* __restrict__ DSP,
                                                       float* __restrict__ dFq, int BH, int T) {
  constexpr int DP = kFP, NDT = DP / 16;
  constexpr int LD = Lds<DP>::PITCH;
  __shared__ __align__(16) float Ks[64 * LD];

  const int NC = (T + 15) >> 4, T16 = 16 * NC;
  const int n_qt = (T + 63) >> 6;
  const int bh = blockIdx.x % BH;
  const int qt = n_qt - 1 - (int)(blockIdx.x / BH);
  const float* FSh = FS + (int64_t)bh * T16 * kFP;
  const int* PSh = PS + (int64_t)bh * T16;
  const int* BSh = BSs + (int64_t)bh * T16;
  const int4* CIh = CI + (int64_t)bh * NC;
  const int64_t rbase = (int64_t)bh * T;

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
  const int lq = lane & 15, g = lane >> 4;
  const int qc = 4 * qt + wave;
  const int qrow = 16 * qc + lq;
  const bool qok = qrow < T;
  const int qpos = qok ? PSh[qrow] : -1;
  const int4 ci = qc < NC ? CIh[qc] : empty_chunk();

  int c0, n_ch;
  bucket_window(BST + bh * 16, BSh[64 * qt], BSh[min(64 * qt + 63, T - 1)], NC, c0, n_ch);
  const int n_kt = (n_ch + 3) >> 2;
  // dS of this head: n_kt_all key tiles x T16 rows x 64
  const int n_kt_all = (T + 63) >> 6;
  const float* dsq = DS + (int64_t)bh * n_kt_all * T16 * 64 + (int64_t)qrow * 64 + 4 * g;

  // the next stage: key feature rows, its live chunks for this wave, and their
  // dS blocks (key chunk c: key tile c / 4 of the dS buffer, columns 16 (c % 4) ..)
  StageInfo nxt;
  ChunkRows<kFP, LD> ks;
  int on_nx = 0;
  float4 dnx[4];
  auto load = [&](int kt) {
    stage_info(CIh, c0, kt, n_ch, NC, nxt);
    ks.load(FSh, nxt.row0, T, tid);
    on_nx = 0;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const bool lv = block_live(ci, nxt.ci[m]);
      on_nx |= lv ? 1 << m : 0;
      const int c = nxt.row0[m] >> 4;
      dnx[m] = (lv && qok) ? *reinterpret_cast<const float4*>(dsq + (int64_t)(c >> 2) * T16 * 64 + 16 * (c & 3))
                           : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  if (n_kt > 0) load(0);

  floatx4 acc[NDT];
#pragma unroll
  for (int dt = 0; dt < NDT; ++dt) acc[dt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int kt = 0; kt < n_kt; ++kt) {
    const int on = on_nx;
    float4 dsv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) dsv[m] = dnx[m];
    __syncthreads();
    ks.store(Ks, tid);
    __syncthreads();
    if (kt + 1 < n_kt) load(kt + 1);
    if (on == 0) continue;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      if (on & (1 << m)) {
        const float d[4] = {dsv[m].x, dsv[m].y, dsv[m].z, dsv[m].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float ka[NDT];
          lds_read_seg<DP, NDT>(Ks, 16 * m + 4 * g + e, lq, ka);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) acc[dt] = mfma4(ka[dt], d[e], acc[dt]);
        }
      }
    }
  }

  if (qok && qpos >= 1) {
    const float dsx = DSP[rbase + qpos];
    const float* fp = F + (rbase + qpos - 1) * kFP + g * (kFP / 4);
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[dt][i] += dsx * fp[NDT * i + dt];
    }
  }
  store_row_frag<kFP, true>(dFq + rbase * kFP, qok ? qpos : T, T, kFP, kFP, g, acc, 1.f);
}

// ------------------------------------------------------------ launchers

size_t wave_sparse_fwd_floats(int B, int H, int T, int) {
  const size_t BH = (size_t)B * H, T16 = (size_t)16 * ((T + 15) / 16), NC = T16 / 16;
  return BH * (2 * T16 + 16 + 4 * NC + T16 * kFP);
}

size_t wave_sparse_bwd_floats(int B, int H, int T, int D) {
  const size_t BH = (size_t)B * H, T16 = (size_t)16 * ((T + 15) / 16);
  return wave_sparse_fwd_floats(B, H, T, D) + BH * (2 * T16 + (size_t)T);
}

size_t wave_sparse_ds_floats(int B, int H, int T) {
  const size_t T16 = (size_t)16 * ((T + 15) / 16);
  return (size_t)B * H * (size_t)((T + 63) / 64) * T16 * 64;
}

namespace {
struct SparseBufs {
  int *perm, *bsort, *bstart;
  int4* ci;
  float *fs, *ls, *dls, *dsp;
};
// Carves the sorted arrays out of ws (wave_sparse_fwd_floats, and for the
// backward wave_sparse_bwd_floats; every part a multiple of 16 bytes).
SparseBufs carve(float* ws, const View& L, bool bwd) {
  const size_t BH = (size_t)L.B * L.H, T16 = (size_t)16 * ((L.T + 15) / 16), NC = T16 / 16;
  SparseBufs s{};
  float* p = ws;
  s.perm = reinterpret_cast<int*>(p);
  p += BH * T16;
  s.bsort = reinterpret_cast<int*>(p);
  p += BH * T16;
  s.bstart = reinterpret_cast<int*>(p);
  p += BH * 16;
  s.ci = reinterpret_cast<int4*>(p);
  p += BH * 4 * NC;
  s.fs = p;
  p += BH * T16 * kFP;
  if (bwd) {
    s.ls = p;
    p += BH * T16;
    s.dls = p;
    p += BH * T16;
    s.dsp = p;
  }
  return s;
}

// Sorts every (b,h)'s positions by bucket and gathers the feature rows and,
// when lse is given, LSE and Delta into sorted order.
hipError_t sort_and_gather(const float* feat, const int* bucket, const float* lse, const float* delta,
                           const SparseBufs& sb, const View& Lv, hipStream_t stream) {
  const int BH = Lv.B * Lv.H, T16 = 16 * ((Lv.T + 15) / 16);
  {
    TimingScope ts("wave_sort", stream);
    hipLaunchKernelGGL(wave_sort_kernel, dim3((unsigned)BH), dim3(kSortThreads), 0, stream, bucket, sb.perm,
                       sb.bsort, sb.bstart, Lv.T, T16);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  TimingScope ts("wave_gather", stream);
  hipLaunchKernelGGL(wave_gather_kernel, dim3((unsigned)(BH * ((T16 + 63) / 64))), dim3(256), 0, stream,
                     (const int*)sb.perm, (const int*)sb.bsort, feat, lse, delta, sb.fs,
                     lse != nullptr ? sb.ls : nullptr, lse != nullptr ? sb.dls : nullptr, sb.ci, Lv);
  return hipGetLastError();
}

#ifndef WHA_SFWD_NW
#define WHA_SFWD_NW 4
#endif
#ifndef WHA_SFWD_DMA
#define WHA_SFWD_DMA 1
#endif
// chunk list of wave_sfwd_reg_kernel: 16 KB of LDS
constexpr int kSfwdMaxChunks = 4096;
template <int DP, bool VEC>
hipError_t sfwd_t(const SparseBufs& sb, const float* feat, const int* bucket, const float* v, float* merged,
                  float* lse, const View& Lv, float cs, hipStream_t stream) {
  constexpr int NW = WHA_SFWD_NW;
  const int n_qt = (Lv.T + 16 * NW - 1) / (16 * NW);
  TimingScope ts("wave_fwd", stream);
  // one wave per 16 sorted queries, when a head's value rows lie within 4 GiB
  // of its first and a row offset is a 24-bit product (32-bit buffer offsets,
  // v_mul_u32_u24) and its chunk list fits in LDS
  const int NC = (Lv.T + 15) / 16;
  if (DP == 64 && VEC && WHA_SFWD_DMA && (uint64_t)Lv.T * (uint64_t)Lv.st * 4u < (1ull << 32) &&
      (uint64_t)Lv.st * 4u < (1u << 24) && Lv.T < (1 << 24) && NC <= kSfwdMaxChunks) {
    const unsigned grid = (unsigned)(NC * Lv.B * Lv.H);
    const size_t lds = (size_t)NC * sizeof(int);
    if (Lv.D == 64)
      hipLaunchKernelGGL(wave_sfwd_reg_kernel<false>, dim3(grid), dim3(64), lds, stream, (const float*)sb.fs,
                         (const int*)sb.perm, (const int*)sb.bsort, (const int4*)sb.ci, (const int*)sb.bstart, feat,
                         bucket, v, merged, lse, Lv, cs);
    else
      hipLaunchKernelGGL(wave_sfwd_reg_kernel<true>, dim3(grid), dim3(64), lds, stream, (const float*)sb.fs,
                         (const int*)sb.perm, (const int*)sb.bsort, (const int4*)sb.ci, (const int*)sb.bstart, feat,
                         bucket, v, merged, lse, Lv, cs);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((wave_sfwd_kernel<DP, VEC, NW>), dim3((unsigned)(n_qt * Lv.B * Lv.H)), dim3(NW * 64), 0, stream,
                     (const float*)sb.fs, (const int*)sb.perm, (const int*)sb.bsort, (const int4*)sb.ci,
                     (const int*)sb.bstart, feat, bucket, v, merged, lse, Lv, cs);
  return hipGetLastError();
}

template <int DP, bool VEC>
hipError_t sdkv_t(const SparseBufs& sb, const float* feat, const int* bucket, const float* v,
                  const float* d_merged, const float* lse, const float* delta, float* dfk, float* dv, float* ds,
                  const View& Lv, float cs, hipStream_t stream) {
  const int n_kt = (Lv.T + 63) / 64;
  TimingScope ts("wave_bwd_dkv", stream);
  // one wave per 16 sorted keys, under the same conditions as the forward's
  const int NC = (Lv.T + 15) / 16;
  if (DP == 64 && VEC && WHA_SFWD_DMA && (uint64_t)Lv.T * (uint64_t)Lv.st * 4u < (1ull << 32) &&
      (uint64_t)Lv.st * 4u < (1u << 24) && Lv.T < (1 << 24) && NC <= kSfwdMaxChunks) {
    const unsigned grid = (unsigned)(NC * Lv.B * Lv.H);
    const size_t lds = (size_t)NC * sizeof(int);
    if (Lv.D == 64)
      hipLaunchKernelGGL(wave_sdkv_dma_kernel<false>, dim3(grid), dim3(64), lds, stream, (const float*)sb.fs,
                         (const float*)sb.ls, (const float*)sb.dls, (const int*)sb.perm, (const int*)sb.bsort,
                         (const int4*)sb.ci, (const int*)sb.bstart, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds,
                         sb.dsp, Lv, cs);
    else
      hipLaunchKernelGGL(wave_sdkv_dma_kernel<true>, dim3(grid), dim3(64), lds, stream, (const float*)sb.fs,
                         (const float*)sb.ls, (const float*)sb.dls, (const int*)sb.perm, (const int*)sb.bsort,
                         (const int4*)sb.ci, (const int*)sb.bstart, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds,
                         sb.dsp, Lv, cs);
    return hipGetLastError();
  }
  hipLaunchKernelGGL((wave_sdkv_kernel<DP, VEC>), dim3((unsigned)(n_kt * Lv.B * Lv.H)), dim3(256), 0, stream,
                     (const float*)sb.fs, (const float*)sb.ls, (const float*)sb.dls, (const int*)sb.perm,
                     (const int*)sb.bsort, (const int4*)sb.ci, (const int*)sb.bstart, feat, bucket, v, d_merged,
                     lse, delta, dfk, dv, ds, sb.dsp, Lv, cs);
  return hipGetLastError();
}
}  // namespace

hipError_t launch_wave_fwd_sparse(const float* feat, const int* bucket, const float* v, float* merged, float* lse,
                                  float* ws, const View& Lv, bool vec, float cs, hipStream_t stream) {
  const SparseBufs sb = carve(ws, Lv, false);
  hipError_t e = sort_and_gather(feat, bucket, nullptr, nullptr, sb, Lv, stream);
  if (e != hipSuccess) return e;
  switch (padded_dim(Lv.D)) {
    case 48:
      return vec ? sfwd_t<48, true>(sb, feat, bucket, v, merged, lse, Lv, cs, stream)
                 : sfwd_t<48, false>(sb, feat, bucket, v, merged, lse, Lv, cs, stream);
    case 64:
      return vec ? sfwd_t<64, true>(sb, feat, bucket, v, merged, lse, Lv, cs, stream)
                 : sfwd_t<64, false>(sb, feat, bucket, v, merged, lse, Lv, cs, stream);
    case 128:
      return vec ? sfwd_t<128, true>(sb, feat, bucket, v, merged, lse, Lv, cs, stream)
                 : sfwd_t<128, false>(sb, feat, bucket, v, merged, lse, Lv, cs, stream);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t launch_wave_bwd_core_sparse(const float* feat, const int* bucket, const float* v, const float* merged,
                                       const float* d_merged, const float* lse, float* delta, float* dfk, float* dfq,
                                       float* dv, float* ds, float* ws, const View& Lv, bool vec, float cs,
                                       hipStream_t stream) {
  hipError_t e = launch_attn_bwd_delta(merged, d_merged, delta, Lv, "wave_bwd_delta", stream);
  if (e != hipSuccess) return e;
  const SparseBufs sb = carve(ws, Lv, true);
  // the queries' LSE and Delta in sorted order (value and dO rows are gathered in the kernel)
  e = sort_and_gather(feat, bucket, lse, delta, sb, Lv, stream);
  if (e != hipSuccess) return e;
  switch (padded_dim(Lv.D)) {
    case 48:
      e = vec ? sdkv_t<48, true>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : sdkv_t<48, false>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    case 64:
      e = vec ? sdkv_t<64, true>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : sdkv_t<64, false>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    case 128:
      e = vec ? sdkv_t<128, true>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream)
              : sdkv_t<128, false>(sb, feat, bucket, v, d_merged, lse, delta, dfk, dv, ds, Lv, cs, stream);
      break;
    default:
      return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  const int n_qt = (Lv.T + 63) / 64;
  TimingScope ts("wave_bwd_dq", stream);
  hipLaunchKernelGGL(wave_sdq_kernel, dim3((unsigned)(n_qt * Lv.B * Lv.H)), dim3(256), 0, stream,
                     (const float*)sb.fs, (const int*)sb.perm, (const int*)sb.bsort, (const int4*)sb.ci,
                     (const int*)sb.bstart, feat, (const float*)ds, (const float*)sb.dsp, dfq, Lv.B * Lv.H, Lv.T);
  return hipGetLastError();
}

}  // namespace wha
