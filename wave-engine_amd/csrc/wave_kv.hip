// KV-cache serving of the wave attention (gfx950): the attention half of the
// reference's prefill and forward_one (src/common/kv_cache.rs:93-356), batched
// over concurrent sequences of different lengths.
//
// Cache per (b,h) and position k (HeadCache, kv_cache.rs:35-41): cos(n phi_k),
// sin(n phi_k), bucket(phi_k), phi_k and the value row.  Decoding one new token
// per sequence scores it against every cached position whose bucket is within
// one of its own (mod 8) or that is the previous position, plus itself with
// score 1 (kv_cache.rs:285-298) -- no content bias, as in the reference's cache
// path -- then appends its entry at index lengths[b].
//
// The decode is a stream over the cache, HBM-bound, so it follows the split-K
// design of the dot-product decode: a block covers one chunk of one (b,h), a
// merge kernel combines the chunks with the self term and writes the appended
// entry.  Within a block the bucket test runs first for the whole chunk and
// only the admitted positions are listed, so the value rows of masked
// positions (about 5/8 of the cache) are never read; 16 lanes then share each
// listed row, each 16-lane group keeping its own online-softmax state.
#include "wha_launch.hpp"

namespace wha {

namespace {
constexpr int kKvThreads = 256;
constexpr int kKvGroups = kKvThreads / 16;
constexpr int kKvUnroll = 4;
constexpr int kKvMaxChunk = 1024;  // keys per block (wave_kv_chunk never exceeds it)

}  // namespace

int wave_kv_chunk(int max_len) {
  int chunk = 1024;
  while (chunk > 256 && (max_len + chunk - 1) / chunk < 8) chunk >>= 1;
  return chunk;
}

// New token per (b,h): qinfo = {cos(n phi), sin(n phi), phi, bucket (as int bits)}.
__global__ __launch_bounds__(256) void wave_kv_query_kernel(const float* __restrict__ proj,
                                                            const float* __restrict__ hraw,
                                                            float4* __restrict__ qinfo, int BH, int H, int P) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= BH) return;
  const int h = i % H;
  const float r = proj[(int64_t)i * P + 0], s = proj[(int64_t)i * P + 1];
  const float phi = wave_phase(s, r);
  const float raw = hraw[h];
  const float n = raw > 20.f ? raw : logf(1.f + expf(raw));
  float sn, cn;
  sincosf(n * phi, &sn, &cn);
  qinfo[i] = make_float4(cn, sn, phi, __int_as_float(wave_phase_bucket(phi)));
}

// One chunk (<= 1024 keys) of one (b,h): partial (max, sum, o[DP]) in the log2
// domain.  Pass 1: every thread tests up to four keys (coalesced bucket and
// cos/sin loads), and the admitted keys with their scores are compacted into
// an LDS list in key order (wave ballots + prefix counts).  Pass 2: 16-lane
// groups stream the value rows of the listed keys only -- all addresses known
// up front, so the loads of a group's four keys in flight are independent.
template <int DP, bool VEC>
__global__ __launch_bounds__(kKvThreads) void wave_kv_split_kernel(const float4* __restrict__ qinfo,
                                                                   const float2* __restrict__ CS,
                                                                   const int* __restrict__ BK,
                                                                   const float* __restrict__ Vc,
                                                                   float* __restrict__ part, KvLens ll, int H,
                                                                   int hd, int cap, int chunk, int n_split) {
  constexpr int NPL = DP / 16;
  constexpr int KPT = kKvMaxChunk / kKvThreads;  // keys tested per thread
  __shared__ int list_k[kKvMaxChunk];
  __shared__ float list_s[kKvMaxChunk];
  __shared__ int wave_cnt[KPT][kKvThreads / 64];
  __shared__ float sm_m[kKvGroups], sm_l[kKvGroups];
  __shared__ float sm_o[kKvGroups][DP];

  const int split = blockIdx.x % n_split;
  const int bh = blockIdx.x / n_split;
  const int b = bh / H;
  const int len = ll.len[b];
  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  const int grp = tid >> 4, sub = tid & 15;
  const int d0 = sub * NPL;
  const float4 q = qinfo[bh];
  const float cq = q.x * kLog2e, sq = q.y * kLog2e;
  const int qb = __float_as_int(q.w);
  const int64_t hb = (int64_t)bh * cap;
  const int k_begin = split * chunk;
  const int k_end = min(len, k_begin + chunk);

  // pass 1: test, score and compact
  bool valid[KPT];
  float score[KPT];
  int pos[KPT];
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    const int key = k_begin + i * kKvThreads + tid;
    const bool in = key < k_end;
    const int kb = in ? BK[hb + key] : 0;
    const float2 c = in ? CS[hb + key] : make_float2(0.f, 0.f);
    valid[i] = in && (wave_bucket_near(kb, qb) || key == len - 1);
    score[i] = cq * c.x + sq * c.y;
    const unsigned long long mask = __ballot(valid[i]);
    pos[i] = __popcll(mask & ((1ull << lane) - 1ull));
    if (lane == 0) wave_cnt[i][wave] = __popcll(mask);
  }
  __syncthreads();
  int n_list = 0;
#pragma unroll
  for (int i = 0; i < KPT; ++i) {
    int before = n_list;
    for (int w = 0; w < kKvThreads / 64; ++w) {
      if (w < wave) before += wave_cnt[i][w];
      n_list += wave_cnt[i][w];
    }
    if (valid[i]) {
      list_k[before + pos[i]] = k_begin + i * kKvThreads + tid;
      list_s[before + pos[i]] = score[i];
    }
  }
  __syncthreads();

  // pass 2: value rows of the listed keys, four in flight per group
  float m = -1e30f, l = 0.f;
  float acc[NPL];
#pragma unroll
  for (int e = 0; e < NPL; ++e) acc[e] = 0.f;
  for (int j0 = grp; j0 < n_list; j0 += kKvGroups * kKvUnroll) {
    float sc[kKvUnroll];
    float vv[kKvUnroll][NPL];
#pragma unroll
    for (int u = 0; u < kKvUnroll; ++u) {
      const int j = j0 + u * kKvGroups;
      const bool in = j < n_list;
      const int key = in ? list_k[j] : 0;
      sc[u] = in ? list_s[j] : -INFINITY;
      const float* vp = Vc + (hb + key) * hd + d0;
      if (VEC && NPL % 4 == 0) {
#pragma unroll
        for (int e4 = 0; e4 < NPL / 4; ++e4) {
          float4 a = make_float4(0.f, 0.f, 0.f, 0.f);
          if (in && d0 + 4 * e4 < hd) {
            // read once: non-temporal (5.7 -> 6.7 TB/s at the 768-dim wave decode)
            const floatx4 t = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(vp + 4 * e4));
            a = make_float4(t[0], t[1], t[2], t[3]);
          }
          vv[u][4 * e4 + 0] = a.x;
          vv[u][4 * e4 + 1] = a.y;
          vv[u][4 * e4 + 2] = a.z;
          vv[u][4 * e4 + 3] = a.w;
        }
      } else {
#pragma unroll
        for (int e = 0; e < NPL; ++e) vv[u][e] = (in && d0 + e < hd) ? vp[e] : 0.f;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < kKvUnroll; ++u) mx = fmaxf(mx, sc[u]);
    const float m_new = fmaxf(m, mx);
    const float alpha = fast_exp2(m - m_new);
    l *= alpha;
#pragma unroll
    for (int e = 0; e < NPL; ++e) acc[e] *= alpha;
#pragma unroll
    for (int u = 0; u < kKvUnroll; ++u) {
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

  // groups that listed no key keep the finite floor and l = 0, o = 0
  float* out = part + ((int64_t)bh * n_split + split) * (DP + 2);
  float M = -1e30f;
#pragma unroll
  for (int gi = 0; gi < kKvGroups; ++gi) M = fmaxf(M, sm_m[gi]);
  if (tid < DP) {
    float o = 0.f;
#pragma unroll
    for (int gi = 0; gi < kKvGroups; ++gi) o += fast_exp2(sm_m[gi] - M) * sm_o[gi][tid];
    out[2 + tid] = o;
  }
  if (tid == 0) {
    float Ls = 0.f;
    for (int gi = 0; gi < kKvGroups; ++gi) Ls += fast_exp2(sm_m[gi] - M) * sm_l[gi];
    out[0] = M;
    out[1] = Ls;
  }
}

// Per (b,h): combine the chunks with the self term (score 1, the new value),
// write the head's slice of merged [B][E], and append the new entry at
// position lengths[b] (checked on the host to be below the capacity).
template <int DP>
__global__ __launch_bounds__(128) void wave_kv_merge_kernel(const float* __restrict__ part,
                                                            const float4* __restrict__ qinfo,
                                                            const float* __restrict__ vnew,
                                                            float* __restrict__ merged, float2* __restrict__ CS,
                                                            int* __restrict__ BK, float* __restrict__ PH,
                                                            float* __restrict__ Vc, KvLens ll, int H, int hd,
                                                            int E, int cap, int chunk, int n_split) {
  const int bh = blockIdx.x;
  const int b = bh / H, h = bh % H;
  const int len = ll.len[b];
  const int nsp = min(n_split, (len + chunk - 1) / chunk);
  const float* p = part + (int64_t)bh * n_split * (DP + 2);
  const float s_self = kLog2e;  // score 1 in log2 units
  float M = s_self;
  for (int s = 0; s < nsp; ++s) M = fmaxf(M, p[s * (DP + 2)]);
  const float w_self = fast_exp2(s_self - M);
  float Ls = w_self;
  for (int s = 0; s < nsp; ++s) Ls += fast_exp2(p[s * (DP + 2)] - M) * p[s * (DP + 2) + 1];
  const float inv = 1.f / Ls;
  const float* vn = vnew + (int64_t)b * E + (int64_t)h * hd;
  float* vdst = Vc + ((int64_t)bh * cap + len) * hd;
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float o = w_self * vn[d];
    for (int s = 0; s < nsp; ++s) o += fast_exp2(p[s * (DP + 2)] - M) * p[s * (DP + 2) + 2 + d];
    merged[(int64_t)b * E + (int64_t)h * hd + d] = o * inv;
    vdst[d] = vn[d];
  }
  if (threadIdx.x == 0) {
    const float4 q = qinfo[bh];
    const int64_t pos = (int64_t)bh * cap + len;
    CS[pos] = make_float2(q.x, q.y);
    BK[pos] = __float_as_int(q.w);
    PH[pos] = q.z;
  }
}

// Prefill: positions [0, T) of the cache from the forward's features, buckets,
// phases and values ([B][T][E]).
__global__ __launch_bounds__(256) void wave_kv_write_kernel(const float* __restrict__ feat,
                                                            const int* __restrict__ bucket,
                                                            const float* __restrict__ phase,
                                                            const float* __restrict__ values,
                                                            float2* __restrict__ CS, int* __restrict__ BK,
                                                            float* __restrict__ PH, float* __restrict__ Vc, int H,
                                                            int T, int hd, int E, int cap, int64_t total) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= total) return;
  const int d = (int)(i % hd);
  const int64_t row = i / hd;  // (b*H + h)*T + t
  const int t = (int)(row % T);
  const int64_t bh = row / T;
  const int b = (int)(bh / H), h = (int)(bh % H);
  const int64_t pos = bh * cap + t;
  Vc[pos * hd + d] = values[((int64_t)b * T + t) * E + (int64_t)h * hd + d];
  if (d == 0) {
    CS[pos] = make_float2(feat[row * kWaveFeatures + 0], feat[row * kWaveFeatures + 1]);
    BK[pos] = bucket[row];
    PH[pos] = phase[row];
  }
}

// Partials for any lengths up to max_len: the chunk is never below 256 keys, so
// ceil(max_len / 256) bounds the split count of every call.
size_t wave_kv_decode_part_floats(int BH, int hd, int max_len) {
  const int n_split = (max_len + 255) / 256;
  return (size_t)BH * (n_split > 0 ? n_split : 1) * (size_t)(padded_dim(hd) + 2);
}

hipError_t launch_wave_kv_write(const float* feat, const int* bucket, const float* phase, const float* values,
                                float* cs, int* bk, float* ph, float* vc, int B, int H, int T, int hd, int E,
                                int cap, hipStream_t stream) {
  const int64_t total = (int64_t)B * H * T * hd;
  TimingScope ts("wave_kv_write", stream);
  hipLaunchKernelGGL(wave_kv_write_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream, feat,
                     bucket, phase, values, reinterpret_cast<float2*>(cs), bk, ph, vc, H, T, hd, E, cap, total);
  return hipGetLastError();
}

template <int DP, bool VEC>
static hipError_t kv_decode_t(const float* proj, const float* hraw, const float* vnew, float* merged, float* cs,
                              int* bk, float* ph, float* vc, float* qinfo, float* part, const KvLens& ll, int B,
                              int H, int P, int hd, int E, int cap, int max_len, hipStream_t stream) {
  const int BH = B * H;
  {
    TimingScope ts("wave_kv_query", stream);
    hipLaunchKernelGGL(wave_kv_query_kernel, dim3((unsigned)((BH + 255) / 256)), dim3(256), 0, stream, proj, hraw,
                       reinterpret_cast<float4*>(qinfo), BH, H, P);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int chunk = wave_kv_chunk(max_len);
  const int n_split = max((max_len + chunk - 1) / chunk, 1);
  {
    TimingScope ts("wave_kv_split", stream);
    hipLaunchKernelGGL((wave_kv_split_kernel<DP, VEC>), dim3((unsigned)(n_split * BH)), dim3(kKvThreads), 0,
                       stream, reinterpret_cast<const float4*>(qinfo), reinterpret_cast<const float2*>(cs),
                       (const int*)bk, (const float*)vc, part, ll, H, hd, cap, chunk, n_split);
  }
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  TimingScope ts("wave_kv_merge", stream);
  hipLaunchKernelGGL((wave_kv_merge_kernel<DP>), dim3((unsigned)BH), dim3(128), 0, stream, (const float*)part,
                     reinterpret_cast<const float4*>(qinfo), vnew, merged, reinterpret_cast<float2*>(cs), bk, ph, vc,
                     ll, H, hd, E, cap, chunk, n_split);
  return hipGetLastError();
}

hipError_t launch_wave_kv_decode(const float* proj, const float* hraw, const float* vnew, float* merged, float* cs,
                                 int* bk, float* ph, float* vc, float* qinfo, float* part, const KvLens& ll, int B,
                                 int H, int P, int hd, int E, int cap, int max_len, bool vec, hipStream_t stream) {
#define WHA_KV(DP)                                                                                            \
  return vec ? kv_decode_t<DP, true>(proj, hraw, vnew, merged, cs, bk, ph, vc, qinfo, part, ll, B, H, P, hd, E, \
                                     cap, max_len, stream)                                                    \
             : kv_decode_t<DP, false>(proj, hraw, vnew, merged, cs, bk, ph, vc, qinfo, part, ll, B, H, P, hd, E, \
                                      cap, max_len, stream)
  switch (padded_dim(hd)) {
    case 48: WHA_KV(48);
    case 64: WHA_KV(64);
    case 128: WHA_KV(128);
    default: return hipErrorInvalidValue;
  }
#undef WHA_KV
}

}  // namespace wha
