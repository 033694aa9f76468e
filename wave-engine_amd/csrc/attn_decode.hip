// Single-token decode against a KV cache (gfx950), split-K over the cache.
//
// Semantics: for each (b,h) one query attends to all T cached keys -- the last
// row of a causal pass with T = cache length, i.e. the row body of
// attention_cpu (reference src/common/compute.rs:380-407) with qi = T-1.  The
// reference itself only has the wave-attention decode of
// src/common/kv_cache.rs:241-356.
//
// The work is a stream over K and V (0.5 FLOP per byte), so the design goal is
// HBM bandwidth, not MFMA: 16 lanes cooperate on one key (each lane owns DP/16
// consecutive d), the dot product is reduced inside the 16-lane row, and each
// 16-lane group keeps its own online-softmax state (running max, sum and
// partial output) over the keys it visits.  A block covers one chunk of keys
// of one (b,h); its 16 groups are merged through LDS into one partial
// (max, sum, o[D]), and decode_merge_kernel combines the chunks.
#include "wha_launch.hpp"

namespace wha {

namespace {
constexpr int kDecThreads = 256;
constexpr int kDecGroups = kDecThreads / 16;  // 16-lane groups per block
constexpr int kDecUnroll = 4;                 // keys in flight per group

inline int decode_chunk(int T) {
  // aim for ~8 K/V chunks of >= 256 keys per (b,h) on long caches
  int chunk = 1024;
  while (chunk > 256 && (T + chunk - 1) / chunk < 8) chunk >>= 1;
  return chunk;
}
inline int decode_splits(int T) { return (T + decode_chunk(T) - 1) / decode_chunk(T); }
}  // namespace

size_t decode_workspace_floats(const View& L) {
  const int DP = padded_dim(L.D);
  return (size_t)L.B * L.H * decode_splits(L.T) * (size_t)(DP + 2);
}

template <int DP, bool VEC>
__global__ __launch_bounds__(kDecThreads) void decode_split_kernel(const float* __restrict__ Qv,
                                                                   const float* __restrict__ Kc,
                                                                   const float* __restrict__ Vc,
                                                                   float* __restrict__ part, View L,
                                                                   int chunk, int n_split,
                                                                   float scale_log2) {
  constexpr int NPL = DP / 16;  // floats per lane
  __shared__ float sm_m[kDecGroups], sm_l[kDecGroups];
  __shared__ float sm_o[kDecGroups][DP];

  const int split = blockIdx.x % n_split;
  const int bh = blockIdx.x / n_split;
  const int b = bh / L.H, h = bh % L.H;
  const int64_t base = (int64_t)b * L.sb + (int64_t)h * L.sh;
  const int tid = threadIdx.x;
  const int grp = tid >> 4, sub = tid & 15;
  const int d0 = sub * NPL;

  float qv[NPL];
  const float* qp = Qv + (int64_t)bh * L.D;
#pragma unroll
  for (int e = 0; e < NPL; ++e) qv[e] = (d0 + e < L.D) ? qp[d0 + e] * scale_log2 : 0.f;

  const int k_begin = split * chunk;
  const int k_end = min(L.T, k_begin + chunk);
  float m = -INFINITY, l = 0.f;
  float acc[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) acc[e] = 0.f;

  for (int k0 = k_begin + grp; k0 < k_end; k0 += kDecGroups * kDecUnroll) {
    float kv[kDecUnroll][NPL], vv[kDecUnroll][NPL];
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      const int key = k0 + u * kDecGroups;
      const float* kp = Kc + base + (int64_t)key * L.st + d0;
      const float* vp = Vc + base + (int64_t)key * L.st + d0;
      if (VEC && NPL % 4 == 0) {
#pragma unroll
        for (int e4 = 0; e4 < NPL / 4; ++e4) {
          float4 a = make_float4(0.f, 0.f, 0.f, 0.f), c = a;
          if (key < k_end && d0 + 4 * e4 < L.D) {
            // read once: non-temporal loads keep the stream from displacing
            // other lines in the caches (6.2 -> 6.9 TB/s at 768-dim decode)
            const floatx4 ta = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(kp + 4 * e4));
            const floatx4 tc = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(vp + 4 * e4));
            a = make_float4(ta[0], ta[1], ta[2], ta[3]);
            c = make_float4(tc[0], tc[1], tc[2], tc[3]);
          }
          kv[u][4 * e4 + 0] = a.x; kv[u][4 * e4 + 1] = a.y; kv[u][4 * e4 + 2] = a.z; kv[u][4 * e4 + 3] = a.w;
          vv[u][4 * e4 + 0] = c.x; vv[u][4 * e4 + 1] = c.y; vv[u][4 * e4 + 2] = c.z; vv[u][4 * e4 + 3] = c.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < NPL; ++e) {
          const bool ok = key < k_end && d0 + e < L.D;
          kv[u][e] = ok ? kp[e] : 0.f;
          vv[u][e] = ok ? vp[e] : 0.f;
        }
      }
    }
    float sc[kDecUnroll];
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      float d = 0.f;
#pragma unroll
      for (int e = 0; e < NPL; ++e) d += qv[e] * kv[u][e];
      d += __shfl_xor(d, 8, 16);
      d += __shfl_xor(d, 4, 16);
      d += __shfl_xor(d, 2, 16);
      d += __shfl_xor(d, 1, 16);
      sc[u] = (k0 + u * kDecGroups < k_end) ? d : -INFINITY;
      mx = fmaxf(mx, sc[u]);
    }
    // the first key of every visited step is valid, so mx is finite unless the
    // scores themselves are not
    const float m_new = fmaxf(m, mx);
    const float alpha = fast_exp2(m - m_new);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < NPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < kDecUnroll; ++u) {
      const float p = fast_exp2(sc[u] - m_new);
      l += p;
#pragma unroll
      for (int e = 0; e < NPL; ++e) acc[e] += p * vv[u][e];
    }
    m = m_new;
  }

  if (sub == 0) {
    sm_m[grp] = m;
    sm_l[grp] = l;
  }
#pragma unroll
  for (int e = 0; e < NPL; ++e) sm_o[grp][d0 + e] = acc[e];
  __syncthreads();

  float* out = part + ((int64_t)bh * n_split + split) * (DP + 2);
  float M = -INFINITY;
#pragma unroll
  for (int gi = 0; gi < kDecGroups; ++gi) M = fmaxf(M, sm_m[gi]);
  // groups that saw no key keep m = -inf and weigh zero
  if (tid < DP) {
    float o = 0.f;
#pragma unroll
    for (int gi = 0; gi < kDecGroups; ++gi)
      if (sm_m[gi] != -INFINITY) o += fast_exp2(sm_m[gi] - M) * sm_o[gi][tid];
    out[2 + tid] = o;
  }
  if (tid == 0) {
    float Ls = 0.f;
    for (int gi = 0; gi < kDecGroups; ++gi)
      if (sm_m[gi] != -INFINITY) Ls += fast_exp2(sm_m[gi] - M) * sm_l[gi];
    out[0] = M;
    out[1] = Ls;
  }
}

template <int DP>
__global__ __launch_bounds__(128) void decode_merge_kernel(const float* __restrict__ part,
                                                           float* __restrict__ O,
                                                           float* __restrict__ LSE, View L,
                                                           int n_split) {
  const int bh = blockIdx.x;
  const float* p = part + (int64_t)bh * n_split * (DP + 2);
  float M = -INFINITY;
  for (int s = 0; s < n_split; ++s) M = fmaxf(M, p[s * (DP + 2)]);
  float Ls = 0.f;
  for (int s = 0; s < n_split; ++s) Ls += fast_exp2(p[s * (DP + 2)] - M) * p[s * (DP + 2) + 1];
  for (int d = threadIdx.x; d < L.D; d += blockDim.x) {
    float o = 0.f;
    for (int s = 0; s < n_split; ++s) o += fast_exp2(p[s * (DP + 2)] - M) * p[s * (DP + 2) + 2 + d];
    O[(int64_t)bh * L.D + d] = o / Ls;
  }
  if (LSE != nullptr && threadIdx.x == 0) LSE[bh] = (M + log2f(Ls)) * kLn2;
}

template <int DP, bool VEC>
static hipError_t decode_t(const float* q, const float* kc, const float* vc, float* o, float* lse,
                           float* ws, const View& L, float scale, hipStream_t stream) {
  const int chunk = decode_chunk(L.T);
  const int n_split = decode_splits(L.T);
  const float sl2 = (float)((double)scale * 1.4426950408889634);
  {
    TimingScope ts("decode_split", stream);
    hipLaunchKernelGGL((decode_split_kernel<DP, VEC>), dim3((unsigned)(n_split * L.B * L.H)),
                       dim3(kDecThreads), 0, stream, q, kc, vc, ws, L, chunk, n_split, sl2);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  {
    TimingScope ts("decode_merge", stream);
    hipLaunchKernelGGL((decode_merge_kernel<DP>), dim3((unsigned)(L.B * L.H)), dim3(128), 0, stream,
                       (const float*)ws, o, lse, L, n_split);
  }
  return hipGetLastError();
}

hipError_t launch_decode(const float* q, const float* kc, const float* vc, float* o, float* lse,
                         float* ws, const View& L, bool vec, float scale, hipStream_t stream) {
  switch (padded_dim(L.D)) {
    case 48:
      return vec ? decode_t<48, true>(q, kc, vc, o, lse, ws, L, scale, stream)
                 : decode_t<48, false>(q, kc, vc, o, lse, ws, L, scale, stream);
    case 64:
      return vec ? decode_t<64, true>(q, kc, vc, o, lse, ws, L, scale, stream)
                 : decode_t<64, false>(q, kc, vc, o, lse, ws, L, scale, stream);
    case 128:
      return vec ? decode_t<128, true>(q, kc, vc, o, lse, ws, L, scale, stream)
                 : decode_t<128, false>(q, kc, vc, o, lse, ws, L, scale, stream);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace wha
