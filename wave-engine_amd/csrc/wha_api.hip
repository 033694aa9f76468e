// C ABI of the gfx950 attention tier: argument validation, error reporting,
// workspace management, host-pointer entry points and optional event timing.
// Declarations and contracts: include/wave_hip_attn.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/wave_hip_attn.h"
#include "wha_launch.hpp"

#ifndef WHA_VERSION
#define WHA_VERSION "0.1.0"
#endif

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(WHA_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

bool aligned16(const void* p) { return p == nullptr || (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Validates a layout; on success fills the kernel view.
int check_layout(const wha_layout* L, wha::View* v, const char* fn) {
  if (L == nullptr) return fail(WHA_ERR_INVALID, "%s: layout is NULL", fn);
  if (L->B <= 0 || L->H <= 0 || L->T <= 0 || L->D <= 0)
    return fail(WHA_ERR_INVALID, "%s: B, H, T, D must be positive (got %d, %d, %d, %d)", fn, L->B, L->H,
                L->T, L->D);
  if (wha::padded_dim(L->D) == 0)
    return fail(WHA_ERR_UNSUPPORTED, "%s: head_dim %d exceeds the supported maximum of 128", fn, L->D);
  if (L->stride_t < L->D || L->stride_h < 0 || L->stride_b < 0)
    return fail(WHA_ERR_INVALID, "%s: invalid strides (b=%lld, h=%lld, t=%lld) for D=%d", fn,
                (long long)L->stride_b, (long long)L->stride_h, (long long)L->stride_t, L->D);
  if ((int64_t)L->B * L->H * L->T > (int64_t)1 << 31)
    return fail(WHA_ERR_UNSUPPORTED, "%s: B*H*T too large", fn);
  // The one layout also describes the outputs (o, dq, dk, dv), so distinct
  // (b, h, t) rows must not overlap: a zero or too-small head/batch stride
  // would let heads overwrite each other's gradients.  Accepted: the
  // dimensions of extent > 1, in increasing stride order, each step at least
  // the span of the smaller ones (rows of D floats) -- this covers [B,H,T,D],
  // [B][T][H*D] and column slices of a fused [B][T][3E] row.
  {
    struct Dim {
      int64_t n, stride;
    } dims[3] = {{L->T, L->stride_t}, {L->H, L->stride_h}, {L->B, L->stride_b}};
    std::sort(dims, dims + 3, [](const Dim& a, const Dim& b) { return a.stride < b.stride; });
    int64_t span = L->D;
    for (const Dim& d : dims) {
      if (d.n <= 1) continue;
      if (d.stride < span)
        return fail(WHA_ERR_INVALID,
                    "%s: strides (b=%lld, h=%lld, t=%lld) make rows of different (b,h,t) overlap for "
                    "B=%d, H=%d, T=%d, D=%d (outputs share the layout and must not alias)",
                    fn, (long long)L->stride_b, (long long)L->stride_h, (long long)L->stride_t, L->B, L->H, L->T,
                    L->D);
      span += d.stride * (d.n - 1);
    }
  }
  v->B = L->B;
  v->H = L->H;
  v->T = L->T;
  v->D = L->D;
  v->sb = L->stride_b;
  v->sh = L->stride_h;
  v->st = L->stride_t;
  return WHA_OK;
}

bool vec_ok(const wha::View& v, std::initializer_list<const void*> ptrs) {
  if (v.D % 4 || v.st % 4 || v.sh % 4 || v.sb % 4) return false;
  for (const void* p : ptrs)
    if (!aligned16(p)) return false;
  return true;
}

int check_scale(float scale, const char* fn) {
  if (!(scale > 0.f) || !std::isfinite(scale))
    return fail(WHA_ERR_INVALID, "%s: scale must be positive and finite (got %g)", fn, (double)scale);
  return WHA_OK;
}

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// ---------------------------------------------------------------- workspace cache
// One growable device buffer per (host thread, device, stream): concurrent
// callers on different threads or streams never share scratch memory.
struct WsEntry {
  int device;
  hipStream_t stream;
  void* ptr;
  size_t bytes;
};
struct WsCache {
  std::vector<WsEntry> entries;
  ~WsCache() {
    for (auto& e : entries)
      if (e.ptr) (void)hipFree(e.ptr);
  }
};
thread_local WsCache g_ws;

int cached_workspace(size_t bytes, hipStream_t stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  for (auto& w : g_ws.entries) {
    if (w.device == dev && w.stream == stream) {
      if (w.bytes < bytes) {
        // the previous user of this buffer was enqueued on the same stream, so
        // freeing after a stream sync is safe
        e = hipStreamSynchronize(stream);
        if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
        (void)hipFree(w.ptr);
        w.ptr = nullptr;
        w.bytes = 0;
        e = hipMalloc(&w.ptr, bytes);
        if (e != hipSuccess) return fail(WHA_ERR_NOMEM, "workspace hipMalloc(%zu) failed", bytes);
        w.bytes = bytes;
      }
      *out = w.ptr;
      return WHA_OK;
    }
  }
  WsEntry w{dev, stream, nullptr, 0};
  e = hipMalloc(&w.ptr, bytes);
  if (e != hipSuccess) return fail(WHA_ERR_NOMEM, "workspace hipMalloc(%zu) failed", bytes);
  w.bytes = bytes;
  g_ws.entries.push_back(w);
  *out = w.ptr;
  return WHA_OK;
}

int resolve_workspace(void* ws, size_t ws_bytes, size_t need, hipStream_t stream, const char* fn,
                      void** out) {
  if (ws == nullptr) return cached_workspace(need, stream, out);
  if (ws_bytes < need)
    return fail(WHA_ERR_WORKSPACE, "%s: workspace of %zu bytes is smaller than the %zu required", fn,
                ws_bytes, need);
  if (!aligned16(ws)) return fail(WHA_ERR_INVALID, "%s: workspace must be 16-byte aligned", fn);
  *out = ws;
  return WHA_OK;
}

// ---------------------------------------------------------------- timing
struct TimingRec {
  std::string name;
  hipEvent_t start, stop;
};
struct TimingState {
  std::mutex mu;
  bool on = false;
  std::vector<TimingRec> pending;
  std::map<std::string, std::pair<double, int64_t>> totals;
  std::vector<hipEvent_t> free_events;  // reused, so a timed launch costs no event creation
};

// An event from the pool (device-scope: the timed kernels share the stream).
hipError_t pooled_event(TimingState& st, hipEvent_t* ev) {
  if (!st.free_events.empty()) {
    *ev = st.free_events.back();
    st.free_events.pop_back();
    return hipSuccess;
  }
  return hipEventCreateWithFlags(ev, hipEventDisableSystemFence);
}
TimingState& timing() {
  static TimingState* s = new TimingState();  // never destroyed: usable during exit
  return *s;
}

int drain_timing_locked(TimingState& st) {
  int rc = WHA_OK;
  for (auto& r : st.pending) {
    hipError_t e = hipEventSynchronize(r.stop);
    float ms = 0.f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, r.start, r.stop);
    if (e != hipSuccess) {
      rc = hip_fail(e, "timing event");
    } else {
      auto& t = st.totals[r.name];
      t.first += ms;
      t.second += 1;
    }
    st.free_events.push_back(r.start);
    st.free_events.push_back(r.stop);
  }
  st.pending.clear();
  return rc;
}

// ---------------------------------------------------------------- host staging
// Per-thread device buffer and stream for the host-pointer entry points.
struct HostStage {
  int device = -1;
  hipStream_t stream = nullptr;
  void* buf = nullptr;
  size_t bytes = 0;
  ~HostStage() {
    if (buf) (void)hipFree(buf);
    if (stream) (void)hipStreamDestroy(stream);
  }
};
thread_local HostStage g_host;

int host_stage(size_t bytes, float** base, hipStream_t* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (g_host.device != dev) {
    if (g_host.buf) (void)hipFree(g_host.buf);
    if (g_host.stream) (void)hipStreamDestroy(g_host.stream);
    g_host.buf = nullptr;
    g_host.bytes = 0;
    g_host.stream = nullptr;
    e = hipStreamCreateWithFlags(&g_host.stream, hipStreamNonBlocking);
    if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
    g_host.device = dev;
  }
  if (g_host.bytes < bytes) {
    if (g_host.buf) {
      (void)hipStreamSynchronize(g_host.stream);
      (void)hipFree(g_host.buf);
    }
    g_host.buf = nullptr;
    g_host.bytes = 0;
    e = hipMalloc(&g_host.buf, bytes);
    if (e != hipSuccess) return fail(WHA_ERR_NOMEM, "host staging hipMalloc(%zu) failed", bytes);
    g_host.bytes = bytes;
  }
  *base = static_cast<float*>(g_host.buf);
  *stream = g_host.stream;
  return WHA_OK;
}

int check_host_seq(const char* fn, int32_t T, int32_t E, int32_t n_head, wha::View* v) {
  if (T <= 0 || E <= 0 || n_head <= 0)
    return fail(WHA_ERR_INVALID, "%s: T, E, n_head must be positive (got %d, %d, %d)", fn, T, E, n_head);
  if (E % n_head != 0)
    return fail(WHA_ERR_INVALID, "%s: n_embd %d is not divisible by n_head %d", fn, E, n_head);
  wha_layout L{1, n_head, T, E / n_head, (int64_t)T * E, (int64_t)(E / n_head), (int64_t)E};
  return check_layout(&L, v, fn);
}

}  // namespace

namespace wha {

TimingScope::TimingScope(const char* name, hipStream_t s) : token(nullptr), stream(s) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  if (!st.on) return;
  TimingRec* r = new TimingRec();
  r->name = name;
  if (pooled_event(st, &r->start) != hipSuccess) {
    delete r;
    return;
  }
  if (pooled_event(st, &r->stop) != hipSuccess) {
    st.free_events.push_back(r->start);
    delete r;
    return;
  }
  if (hipEventRecord(r->start, s) != hipSuccess) {
    st.free_events.push_back(r->start);
    st.free_events.push_back(r->stop);
    delete r;
    return;
  }
  token = r;
}

TimingScope::~TimingScope() {
  if (!token) return;
  TimingRec* r = static_cast<TimingRec*>(token);
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  if (hipEventRecord(r->stop, stream) == hipSuccess) {
    st.pending.push_back(*r);
  } else {
    st.free_events.push_back(r->start);
    st.free_events.push_back(r->stop);
  }
  delete r;
}

}  // namespace wha

extern "C" {

const char* wha_last_error(void) { return g_err; }

const char* wha_version(void) { return WHA_VERSION " gfx950"; }

int wha_attn_fwd(const float* q, const float* k, const float* v, float* o, float* lse,
                 const wha_layout* layout, float scale, void* stream) {
  static const char* fn = "wha_attn_fwd";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k || !v || !o) return fail(WHA_ERR_INVALID, "%s: q, k, v and o must be non-NULL", fn);
  const bool vec = vec_ok(V, {q, k, v, o});
  hipError_t e = wha::launch_attn_fwd(q, k, v, o, lse, V, vec, scale, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_attn_fwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

// Largest dS buffer the fused backward materialises; beyond it (very long
// sequences) the dQ kernel recomputes S and dP instead.
static constexpr size_t kMaxDsBytes = (size_t)8 << 30;

static size_t delta_bytes(const wha_layout* layout) {
  return round256((size_t)layout->B * layout->H * layout->T * sizeof(float));
}

static size_t ds_bytes(const wha_layout* layout) {
  wha::View V{layout->B, layout->H, layout->T, layout->D, 0, 0, 0};
  const size_t n = wha::bwd_ds_floats(V) * sizeof(float);
  return n <= kMaxDsBytes ? round256(n) : 0;
}

// Row statistics of the fused backward (Delta, or the blocked -LSE*log2(e) /
// -Delta pairs the head-dim-64 path uses).
static size_t stats_bytes(const wha_layout* layout) {
  wha::View V{layout->B, layout->H, layout->T, layout->D, 0, 0, 0};
  return round256(wha::bwd_stats_floats(V) * sizeof(float));
}

size_t wha_attn_bwd_workspace_size(const wha_layout* layout) {
  if (!layout || layout->B <= 0 || layout->H <= 0 || layout->T <= 0) return 0;
  return stats_bytes(layout) + ds_bytes(layout);
}

int wha_attn_bwd(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                 const float* lse, float* dq, float* dk, float* dv, void* workspace,
                 size_t workspace_bytes, const wha_layout* layout, float scale, void* stream) {
  static const char* fn = "wha_attn_bwd";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv)
    return fail(WHA_ERR_INVALID, "%s: every tensor pointer must be non-NULL", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, wha_attn_bwd_workspace_size(layout), s, fn, &ws)))
    return rc;
  const bool vec = vec_ok(V, {q, k, v, o, d_o, dq, dk, dv});
  float* delta = static_cast<float*>(ws);
  const size_t dsb = ds_bytes(layout);
  float* ds = dsb ? reinterpret_cast<float*>(static_cast<char*>(ws) + stats_bytes(layout)) : nullptr;
  hipError_t e = wha::launch_attn_bwd(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, V, vec, scale, s);
  if (e != hipSuccess) return hip_fail(e, "wha_attn_bwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

// The kept-scores pair: the forward writes the raw scores of the causal half
// (the dS layout, ds_bytes) and the backward's dK/dV kernel reads them instead
// of recomputing Q K^T.  Covered layouts: the direct-to-LDS head dims with
// 16-byte-aligned strides and a dS buffer within kMaxDsBytes; elsewhere the
// size is 0 and the pair behaves as wha_attn_fwd / wha_attn_bwd.
size_t wha_attn_scores_size(const wha_layout* layout) {
  if (!layout || layout->B <= 0 || layout->H <= 0 || layout->T <= 0 || layout->D <= 0) return 0;
  wha::View V{layout->B, layout->H, layout->T, layout->D, layout->stride_b, layout->stride_h, layout->stride_t};
  const bool strides16 = V.sb % 4 == 0 && V.sh % 4 == 0 && V.st % 4 == 0;
  if (!strides16 || !wha::scores_kept(V, true)) return 0;
  return ds_bytes(layout);
}

// What the last wha_attn_fwd_keep into each score buffer did: whether it
// wrote scores, and for which shape.  wha_attn_bwd_kept reads the scores only
// when this record says they were written for its shape; otherwise it
// recomputes them (always valid, since it has q, k and lse).  This keeps a
// backward from reading scores the forward never wrote, e.g. when the forward
// fell back on unaligned tensors and the backward gets aligned copies of them.
namespace {
struct ScoresRecord {
  bool kept;
  int32_t B, H, T, D;
};
std::mutex g_scores_mu;
std::map<const void*, ScoresRecord> g_scores_rec;
constexpr size_t kMaxScoresRecords = 4096;

void record_scores(const float* scores, bool kept, const wha_layout* L) {
  if (!scores) return;
  std::lock_guard<std::mutex> lk(g_scores_mu);
  // a dropped record only makes a backward recompute, so the table is simply
  // reset when it grows past its bound
  if (g_scores_rec.size() >= kMaxScoresRecords && !g_scores_rec.count(scores)) g_scores_rec.clear();
  g_scores_rec[scores] = ScoresRecord{kept, L->B, L->H, L->T, L->D};
}

bool scores_recorded(const float* scores, const wha_layout* L) {
  if (!scores) return false;
  std::lock_guard<std::mutex> lk(g_scores_mu);
  auto it = g_scores_rec.find(scores);
  if (it == g_scores_rec.end()) return false;
  const ScoresRecord& r = it->second;
  return r.kept && r.B == L->B && r.H == L->H && r.T == L->T && r.D == L->D;
}
}  // namespace

int wha_attn_fwd_keep(const float* q, const float* k, const float* v, float* o, float* lse, float* scores,
                      const wha_layout* layout, float scale, void* stream) {
  static const char* fn = "wha_attn_fwd_keep";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k || !v || !o) return fail(WHA_ERR_INVALID, "%s: q, k, v and o must be non-NULL", fn);
  // Tensors that are not 16-byte aligned run the recompute forward (scores
  // untouched); wha_attn_bwd_kept then falls back as well, since its check
  // includes the same q, k, v, o.
  const bool vec = vec_ok(V, {q, k, v, o});
  const bool keep = wha_attn_scores_size(layout) > 0 && vec;
  if (keep) {
    if (!scores) return fail(WHA_ERR_INVALID, "%s: scores must be non-NULL (wha_attn_scores_size > 0)", fn);
    if (reinterpret_cast<uintptr_t>(scores) & 15)
      return fail(WHA_ERR_INVALID, "%s: scores must be 16-byte aligned", fn);
  }
  hipError_t e = wha::launch_attn_fwd(q, k, v, o, lse, V, vec, scale, static_cast<hipStream_t>(stream),
                                      keep ? scores : nullptr);
  record_scores(scores, keep && e == hipSuccess, layout);
  if (e != hipSuccess) return hip_fail(e, "wha_attn_fwd_keep launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_attn_bwd_kept(const float* q, const float* k, const float* v, const float* o, const float* d_o,
                      const float* lse, const float* scores, float* dq, float* dk, float* dv, void* workspace,
                      size_t workspace_bytes, const wha_layout* layout, float scale, void* stream) {
  static const char* fn = "wha_attn_bwd_kept";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k || !v || !o || !d_o || !lse || !dq || !dk || !dv)
    return fail(WHA_ERR_INVALID, "%s: every tensor pointer must be non-NULL", fn);
  // Unaligned tensors: the recompute backward (the kept scores are not needed).
  const bool vec = vec_ok(V, {q, k, v, o, d_o, dq, dk, dv});
  bool keep = wha_attn_scores_size(layout) > 0 && vec;
  if (keep) {
    if (!scores) return fail(WHA_ERR_INVALID, "%s: scores must be non-NULL (wha_attn_scores_size > 0)", fn);
    if (reinterpret_cast<uintptr_t>(scores) & 15)
      return fail(WHA_ERR_INVALID, "%s: scores must be 16-byte aligned", fn);
    // only scores the forward actually wrote for this shape are read
    keep = scores_recorded(scores, layout);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, wha_attn_bwd_workspace_size(layout), s, fn, &ws)))
    return rc;
  float* delta = static_cast<float*>(ws);
  const size_t dsb = ds_bytes(layout);
  float* ds = dsb ? reinterpret_cast<float*>(static_cast<char*>(ws) + stats_bytes(layout)) : nullptr;
  hipError_t e =
      wha::launch_attn_bwd(q, k, v, o, d_o, lse, dq, dk, dv, delta, ds, V, vec, scale, s, keep ? scores : nullptr);
  if (e != hipSuccess) return hip_fail(e, "wha_attn_bwd_kept launch");
  g_err[0] = 0;
  return WHA_OK;
}

size_t wha_attn_bwd_from_probs_workspace_size(const wha_layout* layout) {
  if (!layout || layout->B <= 0 || layout->H <= 0 || layout->T <= 0) return 0;
  return delta_bytes(layout) + stats_bytes(layout) + ds_bytes(layout);
}

int wha_attn_bwd_from_probs(const float* d_pre_proj, const float* q, const float* k, const float* v,
                            const float* att, float* dq, float* dk, float* dv, void* workspace,
                            size_t workspace_bytes, const wha_layout* layout, float scale,
                            void* stream) {
  static const char* fn = "wha_attn_bwd_from_probs";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!d_pre_proj || !q || !k || !v || !att || !dq || !dk || !dv)
    return fail(WHA_ERR_INVALID, "%s: every tensor pointer must be non-NULL", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, wha_attn_bwd_from_probs_workspace_size(layout), s,
                              fn, &ws)))
    return rc;
  const bool vec = vec_ok(V, {d_pre_proj, q, k, v, dq, dk, dv});
  const size_t dsb = ds_bytes(layout);
  float* stats = reinterpret_cast<float*>(static_cast<char*>(ws) + delta_bytes(layout));
  float* ds = dsb ? reinterpret_cast<float*>(static_cast<char*>(ws) + delta_bytes(layout) + stats_bytes(layout))
                  : nullptr;
  hipError_t e = wha::launch_attn_bwd_probs(d_pre_proj, q, k, v, att, dq, dk, dv, static_cast<float*>(ws),
                                            stats, ds, V, vec, scale, s);
  if (e != hipSuccess) return hip_fail(e, "wha_attn_bwd_from_probs launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_attn_probs_rows(const float* q, const float* k, const float* lse, const int32_t* rows, int32_t n_rows,
                        float* out, const wha_layout* layout, float scale, void* stream) {
  static const char* fn = "wha_attn_probs_rows";
  wha::View V;
  int rc = check_layout(layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k || !lse || !rows || !out) return fail(WHA_ERR_INVALID, "%s: every pointer must be non-NULL", fn);
  if (n_rows < 1 || n_rows > wha::kMaxProbRows)
    return fail(WHA_ERR_INVALID, "%s: n_rows must be in [1, %d] (got %d)", fn, wha::kMaxProbRows, n_rows);
  wha::RowList rl;
  rl.n = n_rows;
  for (int i = 0; i < n_rows; ++i) {
    if (rows[i] < 0 || rows[i] >= V.T)
      return fail(WHA_ERR_INVALID, "%s: rows[%d] = %d is outside [0, %d)", fn, i, rows[i], V.T);
    rl.rows[i] = rows[i];
  }
  hipError_t e = wha::launch_attn_probs_rows(q, k, lse, rl, out, V, scale, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_attn_probs_rows launch");
  g_err[0] = 0;
  return WHA_OK;
}

size_t wha_decode_workspace_size(const wha_layout* layout) {
  wha::View V;
  if (!layout || check_layout(layout, &V, "wha_decode_workspace_size") != WHA_OK) return 0;
  return round256(wha::decode_workspace_floats(V) * sizeof(float));
}

int wha_decode_fwd(const float* q, const float* k_cache, const float* v_cache, float* o, float* lse,
                   void* workspace, size_t workspace_bytes, const wha_layout* cache_layout, float scale,
                   void* stream) {
  static const char* fn = "wha_decode_fwd";
  wha::View V;
  int rc = check_layout(cache_layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  if (!q || !k_cache || !v_cache || !o)
    return fail(WHA_ERR_INVALID, "%s: q, k_cache, v_cache and o must be non-NULL", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, wha_decode_workspace_size(cache_layout), s, fn,
                              &ws)))
    return rc;
  const bool vec = vec_ok(V, {k_cache, v_cache});
  hipError_t e = wha::launch_decode(q, k_cache, v_cache, o, lse, static_cast<float*>(ws), V, vec, scale, s);
  if (e != hipSuccess) return hip_fail(e, "wha_decode_fwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

}  // extern "C"

// ---------------------------------------------------------------- allocation-free decode
// wha_decode_fwd_noalloc keeps its split-K partials in this file-scope device
// array instead of a workspace.  Each GPU holds its own copy for the life of
// the process; host code must use the per-device address from
// hipGetSymbolAddress, never the array's name (a host-side stand-in).
static constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
std::atomic<void*> g_scratch_ptr[kMaxDevices];

// The current device's address of `scratch`, resolved once per device.
int noalloc_scratch(void** out, const char* fn) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(WHA_ERR_UNSUPPORTED, "%s: device index %d is not below %d", fn, dev, kMaxDevices);
  void* p = g_scratch_ptr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    p = g_scratch_ptr[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      g_scratch_ptr[dev].store(p, std::memory_order_release);
    }
  }
  *out = p;
  return WHA_OK;
}
}  // namespace

extern "C" {

int wha_decode_fwd_noalloc(const float* q, const float* k_cache, const float* v_cache, float* o, float* lse,
                           const wha_layout* cache_layout, float scale, void* stream) {
  static const char* fn = "wha_decode_fwd_noalloc";
  wha::View V;
  int rc = check_layout(cache_layout, &V, fn);
  if (rc) return rc;
  if ((rc = check_scale(scale, fn))) return rc;
  // the size limit is checked before the pointers, so a too-large layout is
  // rejected whatever pointers come with it
  const size_t need = wha_decode_workspace_size(cache_layout);
  if (need > kNoAllocScratchBytes)
    return fail(WHA_ERR_WORKSPACE,
                "%s: this cache layout needs %zu bytes of split-K scratch, above the %zu bytes of the static "
                "scratch (use wha_decode_fwd with a workspace)",
                fn, need, kNoAllocScratchBytes);
  if (!q || !k_cache || !v_cache || !o)
    return fail(WHA_ERR_INVALID, "%s: q, k_cache, v_cache and o must be non-NULL", fn);
  void* ws = nullptr;
  if ((rc = noalloc_scratch(&ws, fn))) return rc;
  // every partial the merge kernel reads is written by the split kernel of the
  // same call, so nothing in the scratch needs clearing first
  const bool vec = vec_ok(V, {k_cache, v_cache});
  hipError_t e = wha::launch_decode(q, k_cache, v_cache, o, lse, static_cast<float*>(ws), V, vec, scale,
                                    static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_decode_fwd_noalloc launch");
  g_err[0] = 0;
  return WHA_OK;
}

// ---------------------------------------------------------------- wave attention

static int check_wave_shape(const wha_wave_shape* sh, const char* fn) {
  if (sh == nullptr) return fail(WHA_ERR_INVALID, "%s: shape is NULL", fn);
  if (sh->B <= 0 || sh->T <= 0 || sh->n_embd <= 0 || sh->n_head <= 0)
    return fail(WHA_ERR_INVALID, "%s: B, T, n_embd, n_head must be positive (got %d, %d, %d, %d)", fn, sh->B,
                sh->T, sh->n_embd, sh->n_head);
  if (sh->n_embd % sh->n_head != 0)
    return fail(WHA_ERR_INVALID, "%s: n_embd %d is not divisible by n_head %d", fn, sh->n_embd, sh->n_head);
  if (wha::padded_dim(sh->n_embd / sh->n_head) == 0)
    return fail(WHA_ERR_UNSUPPORTED, "%s: head_dim %d exceeds the supported maximum of 128", fn,
                sh->n_embd / sh->n_head);
  if (sh->content_dim < 0 || sh->content_dim > wha::kWaveFeatures - 2)
    return fail(WHA_ERR_UNSUPPORTED, "%s: content_dim must be in [0, %d] (got %d)", fn, wha::kWaveFeatures - 2,
                sh->content_dim);
  if (sh->n_head > 128)  // the feature kernels stage every head of a position block in LDS
    return fail(WHA_ERR_UNSUPPORTED, "%s: n_head %d exceeds the supported maximum of 128", fn, sh->n_head);
  if ((int64_t)sh->B * sh->n_head * sh->T > ((int64_t)1 << 31) || (int64_t)sh->B * sh->T * sh->n_embd > ((int64_t)1 << 40))
    return fail(WHA_ERR_UNSUPPORTED, "%s: shape too large", fn);
  return WHA_OK;
}

static wha::View wave_view(const wha_wave_shape* sh) {
  const int hd = sh->n_embd / sh->n_head;
  return wha::View{sh->B, sh->n_head, sh->T, hd, (int64_t)sh->T * sh->n_embd, (int64_t)hd, (int64_t)sh->n_embd};
}

static float wave_content_scale(int C) { return C > 0 ? 1.0f / sqrtf((float)C) : 0.0f; }

static int check_wave_cache(const wha_wave_cache* c, const char* fn) {
  if (c == nullptr) return fail(WHA_ERR_INVALID, "%s: cache is NULL", fn);
  if (!c->proj || !c->values || !c->feat || !c->phase || !c->bucket || !c->merged || !c->lse)
    return fail(WHA_ERR_INVALID, "%s: every cache buffer must be non-NULL", fn);
  if (!aligned16(c->feat)) return fail(WHA_ERR_INVALID, "%s: cache->feat must be 16-byte aligned", fn);
  return WHA_OK;
}

static int check_wave_weights(const wha_wave_weights* w, const char* fn) {
  if (w == nullptr) return fail(WHA_ERR_INVALID, "%s: weights is NULL", fn);
  if (!w->harmonic_raw || !w->proj_w || !w->proj_b || !w->v_w || !w->v_b || !w->out_w || !w->out_b)
    return fail(WHA_ERR_INVALID, "%s: every weight pointer must be non-NULL", fn);
  return WHA_OK;
}

// 0: all pairs, 1: bucket-sparse, 2: bucket-sparse from kWaveSparseMinT positions
static std::atomic<int> g_wave_sparse{2};
static constexpr int kWaveSparseMinT = 1024;

int wha_wave_set_bucket_sparse(int mode) {
  if (mode < 0 || mode > 2) return -1;
  return g_wave_sparse.exchange(mode);
}

// The bucket-sparse kernels serve a shape when their score-gradient buffer
// (one [T16][64] block per 64 sorted keys, worst case every pair in the
// window) fits the cap the dense layout has.
static bool wave_sparse_fits(const wha_wave_shape* sh) {
  return wha::wave_sparse_ds_floats(sh->B, sh->n_head, sh->T) * sizeof(float) <= kMaxDsBytes;
}
static bool wave_sparse_on(const wha_wave_shape* sh) {
  const int mode = g_wave_sparse.load(std::memory_order_relaxed);
  return (mode == 1 || (mode == 2 && sh->T >= kWaveSparseMinT)) && wave_sparse_fits(sh);
}

// Scratch of the bucket-sparse forward (sorted operand copies), in bytes; 0
// when the shape never takes that family.
static size_t wave_fwd_sparse_bytes(const wha_wave_shape* sh) {
  if (!wave_sparse_fits(sh)) return 0;
  return round256(wha::wave_sparse_fwd_floats(sh->B, sh->n_head, sh->T, sh->n_embd / sh->n_head) * sizeof(float));
}

size_t wha_wave_fwd_workspace_size(const wha_wave_shape* shape) {
  if (check_wave_shape(shape, "wha_wave_fwd_workspace_size") != WHA_OK) return 0;
  return wave_fwd_sparse_bytes(shape);
}

int wha_wave_fwd(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape, float* out,
                 const wha_wave_cache* cache, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* fn = "wha_wave_fwd";
  int rc;
  if ((rc = check_wave_shape(shape, fn)) || (rc = check_wave_weights(w, fn)) || (rc = check_wave_cache(cache, fn)))
    return rc;
  if (!x || !out) return fail(WHA_ERR_INVALID, "%s: x and out must be non-NULL", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // The scratch is resolved before anything is enqueued, so a too-small
  // workspace leaves every output untouched.
  const bool sparse = wave_sparse_on(shape);
  void* ws = nullptr;
  if (sparse && (rc = resolve_workspace(workspace, workspace_bytes, wave_fwd_sparse_bytes(shape), s, fn, &ws)))
    return rc;
  const int B = shape->B, T = shape->T, E = shape->n_embd, H = shape->n_head, C = shape->content_dim;
  const int hd = E / H, HP = H * (2 + C), M = B * T;
  const wha::View Lv = wave_view(shape);
  const float cs = wave_content_scale(C);
  hipError_t e = wha::launch_linear_fwd(x, E, w->proj_w, w->proj_b, cache->proj, HP, M, HP, E, s);
  if (e == hipSuccess)
    e = wha::launch_linear_fwd_batched(x, E, hd, w->v_w, (int64_t)hd * hd, w->v_b, hd, cache->values, E, hd, M,
                                       hd, hd, H, s);
  if (e == hipSuccess)
    e = wha::launch_wave_features(cache->proj, w->harmonic_raw, cache->feat, cache->phase, cache->bucket, B, H, T,
                                  C, C, s);
  const bool vec = vec_ok(Lv, {cache->values, cache->merged});
  if (e == hipSuccess && sparse) {
    // sorted copies of the operands (the backward sorts again)
    e = wha::launch_wave_fwd_sparse(cache->feat, cache->bucket, cache->values, cache->merged, cache->lse,
                                    static_cast<float*>(ws), Lv, vec, cs, s);
  } else if (e == hipSuccess) {
    e = wha::launch_wave_fwd(cache->feat, cache->bucket, cache->values, cache->merged, cache->lse, Lv, vec, cs, s);
  }
  if (e == hipSuccess) e = wha::launch_linear_fwd(cache->merged, E, w->out_w, w->out_b, out, E, M, E, E, s);
  if (e != hipSuccess) return hip_fail(e, "wha_wave_fwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

// Workspace of wha_wave_bwd, in floats, each part rounded to 64 floats.
struct WaveBwdParts {
  size_t d_merged, delta, ds, dfk, dfq, dv, dproj, hpart, gemm, sorted, total;
};

static WaveBwdParts wave_bwd_parts(const wha_wave_shape* sh) {
  auto r64 = [](size_t n) { return (n + 63) & ~(size_t)63; };
  const size_t B = sh->B, T = sh->T, E = sh->n_embd, H = sh->n_head, P = 2 + sh->content_dim;
  const int64_t M = (int64_t)B * T;
  const int hd = (int)(E / H);
  WaveBwdParts p{};
  p.d_merged = r64(B * T * E);
  p.delta = r64(B * H * T);
  // dS for either kernel family, and the sparse family's sorted operands
  p.ds = r64(wha::bwd_ds_floats(wave_view(sh)));
  if (wave_sparse_fits(sh)) {
    p.ds = std::max(p.ds, r64(wha::wave_sparse_ds_floats((int)B, (int)H, (int)T)));
    p.sorted = r64(wha::wave_sparse_bwd_floats((int)B, (int)H, (int)T, (int)(E / H)));
  }
  p.dfk = r64(B * H * T * wha::kWaveFeatures);
  p.dfq = p.dfk;
  p.dv = r64(B * T * E);
  p.dproj = r64(B * T * H * P);
  p.hpart = r64(B * H * T);
  size_t g = wha::linear_dw_workspace_floats((int)E, (int)E, M);
  g = std::max(g, wha::linear_dw_workspace_floats((int)(H * P), (int)E, M));
  g = std::max(g, wha::linear_dw_workspace_floats(hd, hd, M, (int)H));
  p.gemm = r64(g);
  p.total = p.d_merged + p.delta + p.ds + p.dfk + p.dfq + p.dv + p.dproj + p.hpart + p.gemm + p.sorted;
  return p;
}

size_t wha_wave_bwd_workspace_size(const wha_wave_shape* shape) {
  if (check_wave_shape(shape, "wha_wave_bwd_workspace_size") != WHA_OK) return 0;
  return wave_bwd_parts(shape).total * sizeof(float);
}

int wha_wave_bwd(const float* x, const float* d_out, const wha_wave_weights* w, const wha_wave_shape* shape,
                 const wha_wave_cache* cache, const wha_wave_grads* grads, void* workspace, size_t workspace_bytes,
                 void* stream) {
  static const char* fn = "wha_wave_bwd";
  int rc;
  if ((rc = check_wave_shape(shape, fn)) || (rc = check_wave_weights(w, fn)) || (rc = check_wave_cache(cache, fn)))
    return rc;
  if (!x || !d_out || !grads || !grads->d_x)
    return fail(WHA_ERR_INVALID, "%s: x, d_out, grads and grads->d_x must be non-NULL", fn);
  const float* wg[7] = {grads->d_harmonic_raw, grads->d_proj_w, grads->d_proj_b, grads->d_v_w,
                        grads->d_v_b,          grads->d_out_w,  grads->d_out_b};
  int n_set = 0;
  for (const float* p : wg) n_set += p != nullptr;
  if (n_set != 0 && n_set != 7)
    return fail(WHA_ERR_INVALID, "%s: the weight gradients must be all non-NULL or all NULL", fn);
  const bool full = n_set == 7;
  const WaveBwdParts parts = wave_bwd_parts(shape);
  const bool sparse = wave_sparse_on(shape);
  if (!sparse && wha::bwd_ds_floats(wave_view(shape)) * sizeof(float) > kMaxDsBytes)
    return fail(WHA_ERR_UNSUPPORTED, "%s: B*n_head*T^2 too large for the score-gradient buffer", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* wsv = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, parts.total * sizeof(float), s, fn, &wsv))) return rc;
  float* p = static_cast<float*>(wsv);
  float* d_merged = p;
  p += parts.d_merged;
  float* delta = p;
  p += parts.delta;
  float* ds = p;
  p += parts.ds;
  float* dfk = p;
  p += parts.dfk;
  float* dfq = p;
  p += parts.dfq;
  float* dv = p;
  p += parts.dv;
  float* dproj = p;
  p += parts.dproj;
  float* hpart = p;
  p += parts.hpart;
  float* gws = p;
  p += parts.gemm;
  float* sorted = p;

  const int B = shape->B, T = shape->T, E = shape->n_embd, H = shape->n_head, C = shape->content_dim;
  const int hd = E / H, HP = H * (2 + C), M = B * T;
  const wha::View Lv = wave_view(shape);
  const float cs = wave_content_scale(C);
  const bool vec = vec_ok(Lv, {cache->values, cache->merged, d_merged, dv});
  hipError_t e = wha::launch_linear_bwd_dx(d_out, E, w->out_w, d_merged, E, M, E, E, s);
  if (e == hipSuccess && full)
    e = wha::launch_linear_bwd_dw(d_out, E, cache->merged, E, grads->d_out_w, grads->d_out_b, M, E, E, gws, s);
  if (e == hipSuccess && sparse)
    e = wha::launch_wave_bwd_core_sparse(cache->feat, cache->bucket, cache->values, cache->merged, d_merged,
                                         cache->lse, delta, dfk, dfq, dv, ds, sorted, Lv, vec, cs, s);
  else if (e == hipSuccess)
    e = wha::launch_wave_bwd_core(cache->feat, cache->bucket, cache->values, cache->merged, d_merged, cache->lse,
                                  delta, dfk, dfq, dv, ds, Lv, vec, cs, s);
  if (e == hipSuccess)
    e = wha::launch_wave_feat_bwd(cache->proj, cache->feat, cache->phase, dfq, dfk, w->harmonic_raw, dproj, hpart,
                                  full ? grads->d_harmonic_raw : nullptr, B, H, T, C, cs, s);
  if (e == hipSuccess) e = wha::launch_linear_bwd_dx(dproj, HP, w->proj_w, grads->d_x, E, M, HP, E, s);
  if (e == hipSuccess)
    e = wha::launch_linear_bwd_dx_batched(dv, E, hd, w->v_w, (int64_t)hd * hd, grads->d_x, E, hd, M, hd, hd, H,
                                          true, s);
  if (e == hipSuccess && full)
    e = wha::launch_linear_bwd_dw(dproj, HP, x, E, grads->d_proj_w, grads->d_proj_b, M, HP, E, gws, s);
  if (e == hipSuccess && full)
    e = wha::launch_linear_bwd_dw_batched(dv, E, hd, x, E, hd, grads->d_v_w, (int64_t)hd * hd, grads->d_v_b, M, hd,
                                          hd, H, gws, s);
  if (e != hipSuccess) return hip_fail(e, "wha_wave_bwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_wave_probs_rows(const wha_wave_cache* cache, const wha_wave_shape* shape, const int32_t* rows,
                        int32_t n_rows, float* out, void* stream) {
  static const char* fn = "wha_wave_probs_rows";
  int rc;
  if ((rc = check_wave_shape(shape, fn)) || (rc = check_wave_cache(cache, fn))) return rc;
  if (!rows || !out) return fail(WHA_ERR_INVALID, "%s: rows and out must be non-NULL", fn);
  if (n_rows < 1 || n_rows > wha::kMaxProbRows)
    return fail(WHA_ERR_INVALID, "%s: n_rows must be in [1, %d] (got %d)", fn, wha::kMaxProbRows, n_rows);
  wha::RowList rl;
  rl.n = n_rows;
  for (int i = 0; i < n_rows; ++i) {
    if (rows[i] < 0 || rows[i] >= shape->T)
      return fail(WHA_ERR_INVALID, "%s: rows[%d] = %d is outside [0, %d)", fn, i, rows[i], shape->T);
    rl.rows[i] = rows[i];
  }
  hipError_t e = wha::launch_wave_probs_rows(cache->feat, cache->bucket, cache->lse, rl, out, shape->B,
                                             shape->n_head, shape->T, wave_content_scale(shape->content_dim),
                                             static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_wave_probs_rows launch");
  g_err[0] = 0;
  return WHA_OK;
}

// ---------------------------------------------------------------- wave attention, host forms

namespace {

// Carves 256-byte aligned float segments out of one staging buffer.
struct Carve {
  float* base;
  size_t used;
  float* take(size_t n) {
    float* p = base + used;
    used += round256(n * sizeof(float)) / sizeof(float);
    return p;
  }
};

size_t seg(size_t n) { return round256(n * sizeof(float)); }

struct WaveHostSizes {
  size_t hraw, pw, pb, vw, vb, ow, ob, te, proj, feat, ht;
};

WaveHostSizes wave_host_sizes(int T, int E, int H, int C) {
  const size_t P = 2 + (size_t)C, hd = (size_t)E / H;
  return WaveHostSizes{(size_t)H, (size_t)H * P * E, (size_t)H * P, (size_t)H * hd * hd, (size_t)H * hd,
                       (size_t)E * E, (size_t)E, (size_t)T * E, (size_t)T * H * P,
                       (size_t)H * T * wha::kWaveFeatures, (size_t)H * T};
}

size_t wave_host_weight_bytes(const WaveHostSizes& z) {
  return seg(z.hraw) + seg(z.pw) + seg(z.pb) + seg(z.vw) + seg(z.vb) + seg(z.ow) + seg(z.ob);
}

size_t wave_host_cache_bytes(const WaveHostSizes& z) {
  // proj, values, feat, phase, bucket, merged, lse
  return seg(z.proj) + seg(z.te) + seg(z.feat) + 3 * seg(z.ht) + seg(z.te);
}

// Device copies of the host weights (same layout), enqueued on s.
hipError_t stage_wave_weights(Carve& cv, const wha_wave_weights* w, const WaveHostSizes& z, hipStream_t s,
                              wha_wave_weights* dw) {
  float* d[7] = {cv.take(z.hraw), cv.take(z.pw), cv.take(z.pb), cv.take(z.vw),
                 cv.take(z.vb),   cv.take(z.ow), cv.take(z.ob)};
  const float* h[7] = {w->harmonic_raw, w->proj_w, w->proj_b, w->v_w, w->v_b, w->out_w, w->out_b};
  const size_t n[7] = {z.hraw, z.pw, z.pb, z.vw, z.vb, z.ow, z.ob};
  hipError_t e = hipSuccess;
  for (int i = 0; i < 7 && e == hipSuccess; ++i)
    e = hipMemcpyAsync(d[i], h[i], n[i] * sizeof(float), hipMemcpyHostToDevice, s);
  *dw = wha_wave_weights{d[0], d[1], d[2], d[3], d[4], d[5], d[6]};
  return e;
}

wha_wave_cache carve_wave_cache(Carve& cv, const WaveHostSizes& z) {
  wha_wave_cache c;
  c.proj = cv.take(z.proj);
  c.values = cv.take(z.te);
  c.feat = cv.take(z.feat);
  c.phase = cv.take(z.ht);
  c.bucket = reinterpret_cast<int32_t*>(cv.take(z.ht));
  c.merged = cv.take(z.te);
  c.lse = cv.take(z.ht);
  return c;
}

}  // namespace

int wha_host_wave_attention_forward(const float* x, const wha_wave_weights* w, int32_t T, int32_t E, int32_t H,
                                    int32_t C, float* out, float* phase_out) {
  static const char* fn = "wha_host_wave_attention_forward";
  const wha_wave_shape sh{1, T, E, H, C};
  int rc;
  if ((rc = check_wave_shape(&sh, fn)) || (rc = check_wave_weights(w, fn))) return rc;
  if (!x || !out) return fail(WHA_ERR_INVALID, "%s: x and out must be non-NULL", fn);
  const WaveHostSizes z = wave_host_sizes(T, E, H, C);
  float* base = nullptr;
  hipStream_t s = nullptr;
  const size_t fws_bytes = wha_wave_fwd_workspace_size(&sh);
  if ((rc = host_stage(wave_host_weight_bytes(z) + wave_host_cache_bytes(z) + 2 * seg(z.te) + fws_bytes, &base, &s)))
    return rc;
  Carve cv{base, 0};
  wha_wave_weights dw;
  hipError_t e = stage_wave_weights(cv, w, z, s, &dw);
  float* dx = cv.take(z.te);
  float* dout = cv.take(z.te);
  const wha_wave_cache dc = carve_wave_cache(cv, z);
  void* fws = fws_bytes ? cv.take(fws_bytes / sizeof(float)) : nullptr;
  if (e == hipSuccess) e = hipMemcpyAsync(dx, x, z.te * sizeof(float), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync H2D");
  if ((rc = wha_wave_fwd(dx, &dw, &sh, dout, &dc, fws, fws_bytes, s))) return rc;
  e = hipMemcpyAsync(out, dout, z.te * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess && phase_out)
    e = hipMemcpyAsync(phase_out, dc.phase, z.ht * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync D2H");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_host_wave_attention_backward(const float* x, const float* d_attn_out, const wha_wave_weights* w,
                                     int32_t T, int32_t E, int32_t H, int32_t C, const wha_wave_grads* g) {
  static const char* fn = "wha_host_wave_attention_backward";
  const wha_wave_shape sh{1, T, E, H, C};
  int rc;
  if ((rc = check_wave_shape(&sh, fn)) || (rc = check_wave_weights(w, fn))) return rc;
  if (!x || !d_attn_out || !g || !g->d_x)
    return fail(WHA_ERR_INVALID, "%s: x, d_attn_out, g and g->d_x must be non-NULL", fn);
  float* const hg[7] = {g->d_harmonic_raw, g->d_proj_w, g->d_proj_b, g->d_v_w, g->d_v_b, g->d_out_w, g->d_out_b};
  int n_set = 0;
  for (float* p : hg) n_set += p != nullptr;
  if (n_set != 0 && n_set != 7)
    return fail(WHA_ERR_INVALID, "%s: the weight gradients must be all non-NULL or all NULL", fn);
  const bool full = n_set == 7;
  const WaveHostSizes z = wave_host_sizes(T, E, H, C);
  const size_t ws_bytes = wha_wave_bwd_workspace_size(&sh);
  // the forward's scratch is dead by the time the backward runs: both share it
  const size_t shared_bytes = std::max(ws_bytes, wha_wave_fwd_workspace_size(&sh));
  const size_t grad_bytes = full ? wave_host_weight_bytes(z) : 0;
  float* base = nullptr;
  hipStream_t s = nullptr;
  if ((rc = host_stage(wave_host_weight_bytes(z) + wave_host_cache_bytes(z) + 4 * seg(z.te) + grad_bytes +
                           shared_bytes,
                       &base, &s)))
    return rc;
  Carve cv{base, 0};
  wha_wave_weights dw;
  hipError_t e = stage_wave_weights(cv, w, z, s, &dw);
  float* dx_in = cv.take(z.te);
  float* dout_in = cv.take(z.te);
  float* fwd_out = cv.take(z.te);
  float* d_x = cv.take(z.te);
  const wha_wave_cache dc = carve_wave_cache(cv, z);
  const size_t n[7] = {z.hraw, z.pw, z.pb, z.vw, z.vb, z.ow, z.ob};
  float* dg[7] = {nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  if (full)
    for (int i = 0; i < 7; ++i) dg[i] = cv.take(n[i]);
  void* ws = cv.take(shared_bytes / sizeof(float));
  if (e == hipSuccess) e = hipMemcpyAsync(dx_in, x, z.te * sizeof(float), hipMemcpyHostToDevice, s);
  if (e == hipSuccess) e = hipMemcpyAsync(dout_in, d_attn_out, z.te * sizeof(float), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync H2D");
  if ((rc = wha_wave_fwd(dx_in, &dw, &sh, fwd_out, &dc, ws, shared_bytes, s))) return rc;
  const wha_wave_grads dgr{d_x, dg[0], dg[1], dg[2], dg[3], dg[4], dg[5], dg[6]};
  if ((rc = wha_wave_bwd(dx_in, dout_in, &dw, &sh, &dc, &dgr, ws, ws_bytes, s))) return rc;
  e = hipMemcpyAsync(g->d_x, d_x, z.te * sizeof(float), hipMemcpyDeviceToHost, s);
  if (full)
    for (int i = 0; i < 7 && e == hipSuccess; ++i)
      e = hipMemcpyAsync(hg[i], dg[i], n[i] * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync D2H");
  g_err[0] = 0;
  return WHA_OK;
}

// ---------------------------------------------------------------- wave KV cache

static int check_kv(const wha_wave_kv_cache* kv, const char* fn) {
  if (kv == nullptr) return fail(WHA_ERR_INVALID, "%s: kv cache is NULL", fn);
  if (!kv->cs || !kv->bucket || !kv->phase || !kv->values)
    return fail(WHA_ERR_INVALID, "%s: every kv cache buffer must be non-NULL", fn);
  if (kv->capacity <= 0) return fail(WHA_ERR_INVALID, "%s: capacity must be positive (got %d)", fn, kv->capacity);
  if (!aligned16(kv->values) || (reinterpret_cast<uintptr_t>(kv->cs) & 7u))
    return fail(WHA_ERR_INVALID, "%s: kv->values must be 16-byte and kv->cs 8-byte aligned", fn);
  return WHA_OK;
}

struct KvPrefillParts {
  size_t proj, values, feat, phase, bucket, merged, lse, total;
};

static KvPrefillParts kv_prefill_parts(const wha_wave_shape* sh) {
  auto r64 = [](size_t n) { return (n + 63) & ~(size_t)63; };
  const size_t B = sh->B, T = sh->T, E = sh->n_embd, H = sh->n_head, P = 2 + sh->content_dim;
  KvPrefillParts p{};
  p.proj = r64(B * T * H * P);
  p.values = r64(B * T * E);
  p.feat = r64(B * H * T * wha::kWaveFeatures);
  p.phase = r64(B * H * T);
  p.bucket = r64(B * H * T);
  p.merged = r64(B * T * E);
  p.lse = r64(B * H * T);
  p.total = p.proj + p.values + p.feat + p.phase + p.bucket + p.merged + p.lse;
  return p;
}

size_t wha_wave_kv_prefill_workspace_size(const wha_wave_shape* shape) {
  if (check_wave_shape(shape, "wha_wave_kv_prefill_workspace_size") != WHA_OK) return 0;
  return kv_prefill_parts(shape).total * sizeof(float);
}

int wha_wave_kv_prefill(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape,
                        const wha_wave_kv_cache* kv, float* out, void* workspace, size_t workspace_bytes,
                        void* stream) {
  static const char* fn = "wha_wave_kv_prefill";
  int rc;
  if ((rc = check_wave_shape(shape, fn)) || (rc = check_wave_weights(w, fn)) || (rc = check_kv(kv, fn))) return rc;
  if (!x || !out) return fail(WHA_ERR_INVALID, "%s: x and out must be non-NULL", fn);
  if (shape->T > kv->capacity)
    return fail(WHA_ERR_INVALID, "%s: prompt length %d exceeds the cache capacity %d", fn, shape->T, kv->capacity);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const KvPrefillParts parts = kv_prefill_parts(shape);
  void* wsv = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, parts.total * sizeof(float), s, fn, &wsv))) return rc;
  float* p = static_cast<float*>(wsv);
  float* proj = p;
  p += parts.proj;
  float* values = p;
  p += parts.values;
  float* feat = p;
  p += parts.feat;
  float* phase = p;
  p += parts.phase;
  int* bucket = reinterpret_cast<int*>(p);
  p += parts.bucket;
  float* merged = p;
  p += parts.merged;
  float* lse = p;

  const int B = shape->B, T = shape->T, E = shape->n_embd, H = shape->n_head, C = shape->content_dim;
  const int hd = E / H, HP = H * (2 + C), M = B * T;
  const wha::View Lv = wave_view(shape);
  hipError_t e = wha::launch_linear_fwd(x, E, w->proj_w, w->proj_b, proj, HP, M, HP, E, s);
  if (e == hipSuccess)
    e = wha::launch_linear_fwd_batched(x, E, hd, w->v_w, (int64_t)hd * hd, w->v_b, hd, values, E, hd, M, hd, hd, H,
                                       s);
  if (e == hipSuccess) e = wha::launch_wave_features(proj, w->harmonic_raw, feat, phase, bucket, B, H, T, C, 0, s);
  if (e == hipSuccess)
    e = wha::launch_wave_fwd(feat, bucket, values, merged, lse, Lv, vec_ok(Lv, {values, merged}), 0.f, s);
  if (e == hipSuccess) e = wha::launch_linear_fwd(merged, E, w->out_w, w->out_b, out, E, M, E, E, s);
  if (e == hipSuccess)
    e = wha::launch_wave_kv_write(feat, bucket, phase, values, kv->cs, kv->bucket, kv->phase, kv->values, B, H, T,
                                  hd, E, kv->capacity, s);
  if (e != hipSuccess) return hip_fail(e, "wha_wave_kv_prefill launch");
  g_err[0] = 0;
  return WHA_OK;
}

struct KvDecodeParts {
  size_t proj, vnew, qinfo, merged, part, gemm, total;
};

static KvDecodeParts kv_decode_parts(const wha_wave_shape* sh, int capacity) {
  auto r64 = [](size_t n) { return (n + 63) & ~(size_t)63; };
  const size_t B = sh->B, E = sh->n_embd, H = sh->n_head, P = 2 + sh->content_dim;
  KvDecodeParts p{};
  p.proj = r64(B * H * P);
  p.vnew = r64(B * E);
  p.qinfo = r64(B * H * 4);
  p.merged = r64(B * E);
  p.part = r64(wha::wave_kv_decode_part_floats((int)(B * H), (int)(E / H), capacity));
  const int hd = (int)(E / H);
  size_t g = wha::linear_fwd_workspace_floats((int)B, (int)(H * P), (int)E, 1);
  g = std::max(g, wha::linear_fwd_workspace_floats((int)B, hd, hd, (int)H));
  g = std::max(g, wha::linear_fwd_workspace_floats((int)B, (int)E, (int)E, 1));
  p.gemm = r64(g);
  p.total = p.proj + p.vnew + p.qinfo + p.merged + p.part + p.gemm;
  return p;
}

size_t wha_wave_kv_decode_workspace_size(const wha_wave_shape* shape, int32_t capacity) {
  if (check_wave_shape(shape, "wha_wave_kv_decode_workspace_size") != WHA_OK || capacity <= 0) return 0;
  return kv_decode_parts(shape, capacity).total * sizeof(float);
}

int wha_wave_kv_decode(const float* x, const wha_wave_weights* w, const wha_wave_shape* shape,
                       const wha_wave_kv_cache* kv, const int32_t* lengths, float* out, void* workspace,
                       size_t workspace_bytes, void* stream) {
  static const char* fn = "wha_wave_kv_decode";
  int rc;
  if ((rc = check_wave_shape(shape, fn)) || (rc = check_wave_weights(w, fn)) || (rc = check_kv(kv, fn))) return rc;
  if (!x || !out || !lengths) return fail(WHA_ERR_INVALID, "%s: x, out and lengths must be non-NULL", fn);
  if (shape->T != 1) return fail(WHA_ERR_INVALID, "%s: shape->T must be 1 (one new token per sequence)", fn);
  if (shape->B > wha::kMaxKvBatch)
    return fail(WHA_ERR_UNSUPPORTED, "%s: at most %d sequences per call (got %d)", fn, wha::kMaxKvBatch, shape->B);
  wha::KvLens ll;
  ll.n = shape->B;
  int max_len = 0;
  for (int b = 0; b < shape->B; ++b) {
    if (lengths[b] < 0 || lengths[b] >= kv->capacity)
      return fail(WHA_ERR_INVALID, "%s: lengths[%d] = %d must be in [0, %d) (room to append)", fn, b, lengths[b],
                  kv->capacity);
    ll.len[b] = lengths[b];
    max_len = std::max(max_len, (int)lengths[b]);
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const KvDecodeParts parts = kv_decode_parts(shape, kv->capacity);
  void* wsv = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, parts.total * sizeof(float), s, fn, &wsv))) return rc;
  float* p = static_cast<float*>(wsv);
  float* proj = p;
  p += parts.proj;
  float* vnew = p;
  p += parts.vnew;
  float* qinfo = p;
  p += parts.qinfo;
  float* merged = p;
  p += parts.merged;
  float* part = p;
  p += parts.part;
  float* gws = p;

  const int B = shape->B, E = shape->n_embd, H = shape->n_head, C = shape->content_dim;
  const int hd = E / H, P = 2 + C, HP = H * P;
  const bool vec = hd % 4 == 0 && aligned16(kv->values);
  hipError_t e = wha::launch_linear_fwd_batched(x, E, 0, w->proj_w, 0, w->proj_b, 0, proj, HP, 0, B, HP, E, 1, s, gws);
  if (e == hipSuccess)
    e = wha::launch_linear_fwd_batched(x, E, hd, w->v_w, (int64_t)hd * hd, w->v_b, hd, vnew, E, hd, B, hd, hd, H, s,
                                       gws);
  if (e == hipSuccess)
    e = wha::launch_wave_kv_decode(proj, w->harmonic_raw, vnew, merged, kv->cs, kv->bucket, kv->phase, kv->values,
                                   qinfo, part, ll, B, H, P, hd, E, kv->capacity, max_len, vec, s);
  if (e == hipSuccess)
    e = wha::launch_linear_fwd_batched(merged, E, 0, w->out_w, 0, w->out_b, 0, out, E, 0, B, E, E, 1, s, gws);
  if (e != hipSuccess) return hip_fail(e, "wha_wave_kv_decode launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_host_attention_core_fwd(const float* q, const float* k, const float* v, int32_t T, int32_t E,
                                int32_t n_head, float* o) {
  static const char* fn = "wha_host_attention_core_fwd";
  wha::View V;
  int rc = check_host_seq(fn, T, E, n_head, &V);
  if (rc) return rc;
  if (!q || !k || !v || !o) return fail(WHA_ERR_INVALID, "%s: q, k, v and o must be non-NULL", fn);
  const size_t n = (size_t)T * E;
  const size_t nb = round256(n * sizeof(float)) / sizeof(float);
  float* base = nullptr;
  hipStream_t s = nullptr;
  if ((rc = host_stage(4 * nb * sizeof(float), &base, &s))) return rc;
  float *dq = base, *dk = base + nb, *dv = base + 2 * nb, *dout = base + 3 * nb;
  hipError_t e = hipSuccess;
  const float* srcs[3] = {q, k, v};
  float* dsts[3] = {dq, dk, dv};
  for (int i = 0; i < 3 && e == hipSuccess; ++i)
    e = hipMemcpyAsync(dsts[i], srcs[i], n * sizeof(float), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync H2D");
  const float scale = 1.0f / sqrtf((float)(E / n_head));  // src/common/compute.rs:362
  e = wha::launch_attn_fwd(dq, dk, dv, dout, nullptr, V, vec_ok(V, {dq, dk, dv, dout}), scale, s);
  if (e != hipSuccess) return hip_fail(e, "attention forward launch");
  e = hipMemcpyAsync(o, dout, n * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync D2H");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_host_attention_backward(const float* d_pre_proj, const float* q, const float* k, const float* v,
                                const float* att, int32_t T, int32_t E, int32_t n_head, float* dq,
                                float* dk, float* dv) {
  static const char* fn = "wha_host_attention_backward";
  wha::View V;
  int rc = check_host_seq(fn, T, E, n_head, &V);
  if (rc) return rc;
  if (!d_pre_proj || !q || !k || !v || !att || !dq || !dk || !dv)
    return fail(WHA_ERR_INVALID, "%s: every pointer must be non-NULL", fn);
  const size_t n = (size_t)T * E;
  const size_t nb = round256(n * sizeof(float)) / sizeof(float);
  const size_t na = round256((size_t)n_head * T * T * sizeof(float)) / sizeof(float);
  // the device entry's workspace (Delta, the statistics blocks and dS of the
  // direct-to-LDS kernels) for the staged [T][E] sequence
  const wha_layout sl{1, n_head, T, E / n_head, (int64_t)T * E, (int64_t)(E / n_head), (int64_t)E};
  const size_t ws_bytes = wha_attn_bwd_from_probs_workspace_size(&sl);
  float* base = nullptr;
  hipStream_t s = nullptr;
  if ((rc = host_stage((7 * nb + na) * sizeof(float) + ws_bytes, &base, &s))) return rc;
  float* d_do = base;
  float* d_q = base + nb;
  float* d_k = base + 2 * nb;
  float* d_v = base + 3 * nb;
  float* d_dq = base + 4 * nb;
  float* d_dk = base + 5 * nb;
  float* d_dv = base + 6 * nb;
  float* d_att = base + 7 * nb;
  float* d_delta = d_att + na;
  float* d_stats = reinterpret_cast<float*>(reinterpret_cast<char*>(d_delta) + delta_bytes(&sl));
  float* d_ds = ds_bytes(&sl) ? reinterpret_cast<float*>(reinterpret_cast<char*>(d_stats) + stats_bytes(&sl))
                              : nullptr;
  hipError_t e = hipSuccess;
  const float* srcs[4] = {d_pre_proj, q, k, v};
  float* dsts[4] = {d_do, d_q, d_k, d_v};
  for (int i = 0; i < 4 && e == hipSuccess; ++i)
    e = hipMemcpyAsync(dsts[i], srcs[i], n * sizeof(float), hipMemcpyHostToDevice, s);
  if (e == hipSuccess)
    e = hipMemcpyAsync(d_att, att, (size_t)n_head * T * T * sizeof(float), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync H2D");
  const float scale = 1.0f / sqrtf((float)(E / n_head));  // src/cpu/backward.rs:326
  e = wha::launch_attn_bwd_probs(d_do, d_q, d_k, d_v, d_att, d_dq, d_dk, d_dv, d_delta, d_stats, d_ds, V,
                                 vec_ok(V, {d_do, d_q, d_k, d_v, d_dq, d_dk, d_dv}), scale, s);
  if (e != hipSuccess) return hip_fail(e, "attention backward launch");
  float* outs[3] = {dq, dk, dv};
  const float* douts[3] = {d_dq, d_dk, d_dv};
  for (int i = 0; i < 3 && e == hipSuccess; ++i)
    e = hipMemcpyAsync(outs[i], douts[i], n * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync D2H");
  g_err[0] = 0;
  return WHA_OK;
}

}  // extern "C"

namespace {

int check_linear(const char* fn, int64_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0)
    return fail(WHA_ERR_INVALID, "%s: M, N, K must be positive (got %lld, %d, %d)", fn, (long long)M, N, K);
  if (M > (int64_t)65535 * 128)
    return fail(WHA_ERR_UNSUPPORTED, "%s: M = %lld rows exceeds %d", fn, (long long)M, 65535 * 128);
  return WHA_OK;
}

}  // namespace

extern "C" {

int wha_linear_fwd(const float* x, int64_t ldx, const float* w, const float* b, float* y, int64_t ldy, int64_t M,
                   int32_t N, int32_t K, void* stream) {
  static const char* fn = "wha_linear_fwd";
  int rc = check_linear(fn, M, N, K);
  if (rc) return rc;
  if (!x || !w || !y) return fail(WHA_ERR_INVALID, "%s: x, w and y must be non-NULL", fn);
  if (ldx < K || ldy < N) return fail(WHA_ERR_INVALID, "%s: ldx must be >= K and ldy >= N", fn);
  hipError_t e = wha::launch_linear_fwd(x, ldx, w, b, y, ldy, (int)M, N, K, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_linear_fwd launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_linear_bwd_dx(const float* dy, int64_t lddy, const float* w, float* dx, int64_t lddx, int64_t M, int32_t N,
                      int32_t K, void* stream) {
  static const char* fn = "wha_linear_bwd_dx";
  int rc = check_linear(fn, M, N, K);
  if (rc) return rc;
  if (!dy || !w || !dx) return fail(WHA_ERR_INVALID, "%s: dy, w and dx must be non-NULL", fn);
  if (lddy < N || lddx < K) return fail(WHA_ERR_INVALID, "%s: lddy must be >= N and lddx >= K", fn);
  hipError_t e = wha::launch_linear_bwd_dx(dy, lddy, w, dx, lddx, (int)M, N, K, static_cast<hipStream_t>(stream));
  if (e != hipSuccess) return hip_fail(e, "wha_linear_bwd_dx launch");
  g_err[0] = 0;
  return WHA_OK;
}

size_t wha_linear_bwd_dw_workspace_size(int64_t M, int32_t N, int32_t K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return round256(wha::linear_dw_workspace_floats(N, K, M) * sizeof(float));
}

int wha_linear_bwd_dw(const float* dy, int64_t lddy, const float* x, int64_t ldx, float* dw, float* db, int64_t M,
                      int32_t N, int32_t K, void* workspace, size_t workspace_bytes, void* stream) {
  static const char* fn = "wha_linear_bwd_dw";
  int rc = check_linear(fn, M, N, K);
  if (rc) return rc;
  if (!dy || !x || !dw) return fail(WHA_ERR_INVALID, "%s: dy, x and dw must be non-NULL", fn);
  if (lddy < N || ldx < K) return fail(WHA_ERR_INVALID, "%s: lddy must be >= N and ldx >= K", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if ((rc = resolve_workspace(workspace, workspace_bytes, wha_linear_bwd_dw_workspace_size(M, N, K), s, fn, &ws)))
    return rc;
  hipError_t e = wha::launch_linear_bwd_dw(dy, lddy, x, ldx, dw, db, (int)M, N, K, static_cast<float*>(ws), s);
  if (e != hipSuccess) return hip_fail(e, "wha_linear_bwd_dw launch");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_host_attention(const float* x, const float* c_attn_w, const float* c_attn_b, const float* c_proj_w,
                       const float* c_proj_b, int32_t T, int32_t E, int32_t n_head, float* out) {
  static const char* fn = "wha_host_attention";
  wha::View V;
  int rc = check_host_seq(fn, T, E, n_head, &V);
  if (rc) return rc;
  if (!x || !c_attn_w || !c_attn_b || !c_proj_w || !c_proj_b || !out)
    return fail(WHA_ERR_INVALID, "%s: every pointer must be non-NULL", fn);
  const size_t E3 = (size_t)3 * E;
  auto fl = [](size_t n) { return round256(n * sizeof(float)) / sizeof(float); };
  const size_t n_x = fl((size_t)T * E), n_wa = fl(E3 * E), n_ba = fl(E3), n_wp = fl((size_t)E * E), n_bp = fl(E);
  const size_t n_qkv = fl((size_t)T * E3);
  float* base = nullptr;
  hipStream_t s = nullptr;
  if ((rc = host_stage((2 * n_x + n_wa + n_ba + n_wp + n_bp + 2 * n_qkv) * sizeof(float), &base, &s))) return rc;
  float* d_x = base;
  float* d_wa = d_x + n_x;
  float* d_ba = d_wa + n_wa;
  float* d_wp = d_ba + n_ba;
  float* d_bp = d_wp + n_wp;
  float* d_qkv = d_bp + n_bp;
  float* d_o = d_qkv + n_qkv;  // [T][3E] pitch, first E columns used
  float* d_out = d_o + n_qkv;
  struct Copy { float* dst; const float* src; size_t n; } copies[] = {
      {d_x, x, (size_t)T * E}, {d_wa, c_attn_w, E3 * E}, {d_ba, c_attn_b, E3},
      {d_wp, c_proj_w, (size_t)E * E}, {d_bp, c_proj_b, (size_t)E}};
  hipError_t e = hipSuccess;
  for (const Copy& c : copies)
    if (e == hipSuccess) e = hipMemcpyAsync(c.dst, c.src, c.n * sizeof(float), hipMemcpyHostToDevice, s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync H2D");
  // qkv = c_attn(x)  (src/common/compute.rs:368-375)
  e = wha::launch_linear_fwd(d_x, E, d_wa, d_ba, d_qkv, (int64_t)E3, T, (int)E3, E, s);
  if (e != hipSuccess) return hip_fail(e, "c_attn launch");
  // core on the q, k, v column blocks of qkv, read in place
  const int D = E / n_head;
  wha::View Vq{1, n_head, T, D, (int64_t)T * (int64_t)E3, D, (int64_t)E3};
  const float scale = 1.0f / sqrtf((float)D);  // src/common/compute.rs:362
  e = wha::launch_attn_fwd(d_qkv, d_qkv + E, d_qkv + 2 * E, d_o, nullptr, Vq,
                           vec_ok(Vq, {d_qkv, d_qkv + E, d_qkv + 2 * E, d_o}), scale, s);
  if (e != hipSuccess) return hip_fail(e, "attention core launch");
  // out = c_proj(o)  (:411-413)
  e = wha::launch_linear_fwd(d_o, (int64_t)E3, d_wp, d_bp, d_out, E, T, E, E, s);
  if (e != hipSuccess) return hip_fail(e, "c_proj launch");
  e = hipMemcpyAsync(out, d_out, (size_t)T * E * sizeof(float), hipMemcpyDeviceToHost, s);
  if (e == hipSuccess) e = hipStreamSynchronize(s);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync D2H");
  g_err[0] = 0;
  return WHA_OK;
}

int wha_timing_enable(int on) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  st.on = on != 0;
  return WHA_OK;
}

int wha_timing_reset(void) {
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  int rc = drain_timing_locked(st);
  st.totals.clear();
  return rc;
}

int wha_timing_read(const char* kernel, double* total_ms, int64_t* launches) {
  if (!kernel || !total_ms || !launches) return fail(WHA_ERR_INVALID, "wha_timing_read: NULL argument");
  TimingState& st = timing();
  std::lock_guard<std::mutex> lk(st.mu);
  int rc = drain_timing_locked(st);
  auto it = st.totals.find(kernel);
  *total_ms = it == st.totals.end() ? 0.0 : it->second.first;
  *launches = it == st.totals.end() ? 0 : it->second.second;
  return rc;
}

}  // extern "C"
