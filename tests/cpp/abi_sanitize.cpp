// Host AddressSanitizer / UndefinedBehaviorSanitizer run of the C ABI's host
// layer (argument validation, size arithmetic, error strings, the seeded
// generator's threads, the timing bookkeeping), built with the host code
// instrumented (-Xarch_host -fsanitize=...; device code is not) and run where
// no GPU is visible.  Every call here must be rejected, or be pure host work,
// before any device access.  Built and run by tests/test_sanitizers.py
// (Makefile target `sanitize`); exit status 0 and no sanitizer report means
// clean.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/wave_hip_attn.h"

static int g_fail = 0;

static void expect(bool ok, const char* what) {
  if (!ok) {
    std::fprintf(stderr, "FAILED: %s (last error: %s)\n", what, wha_last_error());
    g_fail = 1;
  }
}

static wha_layout bhtd(int B, int H, int T, int D) {
  return wha_layout{B, H, T, D, (int64_t)H * T * D, (int64_t)T * D, D};
}

int main() {
  // made-up device addresses: validation must reject every call below first
  float* p = reinterpret_cast<float*>(uintptr_t(1) << 20);
  const float* cp = p;
  expect(std::strstr(wha_version(), "gfx950") != nullptr, "version");

  // layouts
  expect(wha_attn_fwd(cp, cp, cp, p, nullptr, nullptr, 0.125f, nullptr) == WHA_ERR_INVALID, "NULL layout");
  wha_layout bad[] = {bhtd(0, 1, 1, 64), bhtd(1, -1, 1, 64), bhtd(1, 1, 0, 64), bhtd(1, 1, 1, 0)};
  for (auto& L : bad) expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "dims");
  wha_layout big_d = bhtd(1, 1, 4, 129);
  expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &big_d, 0.125f, nullptr) == WHA_ERR_UNSUPPORTED, "D > 128");
  wha_layout st = bhtd(1, 2, 16, 64);
  st.stride_t = 32;
  expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &st, 0.125f, nullptr) == WHA_ERR_INVALID, "stride_t < D");
  const int64_t overl[][3] = {{2 * 16 * 64, 0, 64}, {0, 16 * 64, 64}, {2 * 16 * 64, 64, 64}, {16 * 64, 16 * 64, 64}};
  for (auto& s : overl) {
    wha_layout L = bhtd(2, 2, 16, 64);
    L.stride_b = s[0];
    L.stride_h = s[1];
    L.stride_t = s[2];
    expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "overlapping strides");
    expect(std::strstr(wha_last_error(), "overlap") != nullptr, "overlap message");
  }
  wha_layout huge = bhtd(1 << 16, 1 << 10, 1 << 10, 64);
  expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &huge, 0.125f, nullptr) == WHA_ERR_UNSUPPORTED, "B*H*T too large");

  // scale and NULL pointers, every device entry point
  wha_layout L = bhtd(2, 3, 100, 64);
  const float scales[] = {0.f, -1.f, INFINITY, NAN};
  for (float s : scales) expect(wha_attn_fwd(cp, cp, cp, p, nullptr, &L, s, nullptr) == WHA_ERR_INVALID, "scale");
  expect(wha_attn_fwd(nullptr, cp, cp, p, nullptr, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "fwd NULL");
  expect(wha_attn_bwd(nullptr, cp, cp, cp, cp, cp, p, p, p, nullptr, 0, &L, 0.125f, nullptr) == WHA_ERR_INVALID,
         "bwd NULL");
  // 256 tiles of 64 rows: not a small problem, so the kept pair keeps scores and checks the buffer
  wha_layout Lk = bhtd(8, 16, 128, 64);
  expect(wha_attn_fwd_keep(cp, cp, cp, p, p, nullptr, &Lk, 0.125f, nullptr) == WHA_ERR_INVALID, "keep NULL scores");
  float* odd = reinterpret_cast<float*>((uintptr_t(1) << 20) + 4);
  expect(wha_attn_fwd_keep(cp, cp, cp, p, p, odd, &Lk, 0.125f, nullptr) == WHA_ERR_INVALID, "keep odd scores");
  expect(wha_attn_bwd_kept(cp, cp, cp, cp, cp, cp, nullptr, p, p, p, nullptr, 0, &Lk, 0.125f, nullptr) ==
             WHA_ERR_INVALID,
         "kept NULL scores");
  expect(wha_attn_bwd_from_probs(nullptr, cp, cp, cp, cp, p, p, p, nullptr, 0, &L, 0.125f, nullptr) ==
             WHA_ERR_INVALID,
         "from_probs NULL");
  expect(wha_attn_bwd(cp, cp, cp, cp, cp, cp, p, p, p, p, 16, &L, 0.125f, nullptr) == WHA_ERR_WORKSPACE,
         "small workspace");
  expect(wha_decode_fwd(nullptr, cp, cp, p, nullptr, nullptr, 0, &L, 0.125f, nullptr) == WHA_ERR_INVALID,
         "decode NULL");
  wha_layout long_cache = bhtd(64, 12, 1 << 17, 64);
  expect(wha_decode_fwd_noalloc(nullptr, nullptr, nullptr, nullptr, nullptr, &long_cache, 0.125f, nullptr) ==
             WHA_ERR_WORKSPACE,
         "noalloc beyond its scratch");
  int32_t rows[2] = {3, 100};
  expect(wha_attn_probs_rows(cp, cp, cp, rows, 2, p, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "row outside T");
  expect(wha_attn_probs_rows(cp, cp, cp, rows, 0, p, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "no rows");
  expect(wha_attn_probs_rows(cp, cp, cp, rows, 257, p, &L, 0.125f, nullptr) == WHA_ERR_INVALID, "too many rows");

  // size functions: valid and invalid layouts
  const wha_layout sizes[] = {bhtd(8, 12, 1024, 64), bhtd(4, 32, 2048, 128), bhtd(4, 4, 256, 42), bhtd(1, 1, 1, 8),
                              bhtd(16, 8, 512, 48), bhtd(0, 1, 1, 1)};
  for (const auto& S : sizes) {
    volatile size_t a = wha_attn_bwd_workspace_size(&S) + wha_attn_scores_size(&S) +
                        wha_attn_bwd_from_probs_workspace_size(&S) + wha_decode_workspace_size(&S);
    (void)a;
  }
  expect(wha_attn_bwd_workspace_size(nullptr) == 0 && wha_attn_scores_size(nullptr) == 0, "NULL size layout");

  // projections
  expect(wha_linear_fwd(cp, 8, cp, nullptr, p, 8, 0, 8, 8, nullptr) == WHA_ERR_INVALID, "linear M = 0");
  expect(wha_linear_fwd(nullptr, 8, cp, nullptr, p, 8, 4, 8, 8, nullptr) == WHA_ERR_INVALID, "linear NULL");
  expect(wha_linear_bwd_dx(cp, 8, cp, p, 4, 4, 8, 8, nullptr) == WHA_ERR_INVALID, "dx ldx < K");
  expect(wha_linear_bwd_dw(cp, 8, cp, 8, nullptr, nullptr, 4, 8, 8, nullptr, 0, nullptr) == WHA_ERR_INVALID,
         "dw NULL");
  volatile size_t lw = wha_linear_bwd_dw_workspace_size(8192, 2304, 768) + wha_linear_bwd_dw_workspace_size(1, 1, 1);
  (void)lw;

  // host entry points
  std::vector<float> h(64, 0.f);
  expect(wha_host_attention_core_fwd(h.data(), h.data(), h.data(), 4, 10, 3, h.data()) == WHA_ERR_INVALID,
         "host E % H");
  expect(wha_host_attention_backward(h.data(), h.data(), h.data(), h.data(), h.data(), 4, 8, 0, h.data(), h.data(),
                                     h.data()) == WHA_ERR_INVALID,
         "host n_head 0");
  expect(wha_host_attention(h.data(), h.data(), h.data(), h.data(), h.data(), 0, 8, 2, h.data()) == WHA_ERR_INVALID,
         "host T 0");

  // wave attention and KV cache validation
  wha_wave_weights w{cp, cp, cp, cp, cp, cp, cp};
  wha_wave_cache c{p, p, p, p, reinterpret_cast<int32_t*>(p), p, p};
  wha_wave_shape wsh[] = {{1, 8, 63, 2, 16}, {1, 8, 64, 2, 31}, {1, 8, 258, 1, 16}, {1, 0, 64, 2, 16},
                          {1, 8, 258, 129, 0}};
  for (auto& s : wsh) expect(wha_wave_fwd(cp, &w, &s, p, &c, nullptr, 0, nullptr) != WHA_OK, "wave shape");
  wha_wave_shape wbig{2, 1024, 768, 12, 16};
  expect(wha_wave_fwd(cp, &w, &wbig, p, &c, p, wha_wave_fwd_workspace_size(&wbig) - 16, nullptr) ==
             WHA_ERR_WORKSPACE,
         "wave forward workspace too small");
  wha_wave_shape ok{1, 8, 64, 2, 16};
  wha_wave_grads some{p, p, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
  expect(wha_wave_bwd(cp, cp, &w, &ok, &c, &some, nullptr, 0, nullptr) == WHA_ERR_INVALID, "wave grads mix");
  int32_t wrow = 8;
  expect(wha_wave_probs_rows(&c, &ok, &wrow, 1, p, nullptr) == WHA_ERR_INVALID, "wave row outside T");
  wha_wave_kv_cache kv{p, reinterpret_cast<int32_t*>(p), p, p, 16};
  wha_wave_shape dec{2, 1, 64, 2, 16};
  int32_t lens[2] = {3, 16};
  expect(wha_wave_kv_decode(cp, &w, &dec, &kv, lens, p, nullptr, 0, nullptr) == WHA_ERR_INVALID, "kv full");
  wha_wave_shape pre{1, 17, 64, 2, 16};
  expect(wha_wave_kv_prefill(cp, &w, &pre, &kv, p, nullptr, 0, nullptr) == WHA_ERR_INVALID, "prompt > capacity");
  volatile size_t ws = wha_wave_bwd_workspace_size(&ok) + wha_wave_kv_prefill_workspace_size(&ok) +
                       wha_wave_kv_decode_workspace_size(&dec, 8192) + wha_wave_kv_decode_workspace_size(&dec, 0);
  (void)ws;

  // the seeded generator: threaded output equals the sequential stream
  const size_t n = (size_t)5 << 20;
  std::vector<float> a(n), b(n);
  uint64_t s1 = 42, s2 = 42;
  expect(wha_synth_normal(&s1, a.data(), n, 0.125, 1) == 0, "synth 1 thread");
  expect(wha_synth_normal(&s2, b.data(), n, 0.125, 8) == 0, "synth 8 threads");
  expect(s1 == s2 && std::memcmp(a.data(), b.data(), n * sizeof(float)) == 0, "threaded stream equals sequential");
  uint64_t zero = 0;
  expect(wha_synth_normal(&zero, a.data(), 4, 1.0, 1) == -1, "zero state");

  // timing bookkeeping from several threads (no device work recorded)
  std::vector<std::thread> th;
  for (int t = 0; t < 4; ++t)
    th.emplace_back([] {
      double ms = 0;
      int64_t nl = 0;
      wha_timing_reset();
      wha_timing_read("attn_fwd", &ms, &nl);
      if (wha_timing_read(nullptr, &ms, &nl) != WHA_ERR_INVALID) g_fail = 1;
    });
  for (auto& t : th) t.join();

  std::printf(g_fail ? "abi_sanitize: FAILED\n" : "abi_sanitize: OK\n");
  return g_fail;
}
