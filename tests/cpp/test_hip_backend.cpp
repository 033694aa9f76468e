// Tests of the C++ host mirror (wave-engine_amd/csrc/hip_backend.hpp) on the GPU,
// written in the shape of the reference's in-file #[test] functions
// (e.g. src/common/math/attn_backward.rs:352-379).  The CPU oracle
// (oracle/liboracle.so, test infrastructure) is the checker.
// Run by tests/test_gpu_host.py; needs an MI355X.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <functional>
#include <string>
#include <thread>
#include <vector>

#include "../../wave-engine_amd/csrc/hip_backend.hpp"

extern "C" {
void wao_fill_normal(uint64_t* state, float* out, size_t n, double stddev);
void wao_attention_core_fwd_f32(const float* q, const float* k, const float* v, int T, int E, int H,
                                float* out, float* att_out, float* lse_out);
void wao_attention_full_f32(const float* x, const float* wa, const float* ba, const float* wp, const float* bp,
                            int T, int E, int H, float* out);
void wao_attention_backward_f32(const float* d_pre_proj, const float* q, const float* k, const float* v,
                                const float* att, int T, int E, int H, float* dq, float* dk, float* dv);
void wao_wave_fwd_f32(const float* x, int T, int E, int H, int C, const float* hraw, const float* proj_w,
                      const float* proj_b, const float* v_w, const float* v_b, const float* out_w, const float* out_b,
                      const float* phase_in, float* out, float* merged_out, float* att_out, float* phase_out,
                      float* rs_out, float* content_out, float* values_out, float* lse_out);
void wao_wave_bwd_f32(const float* x, int T, int E, int H, int C, const float* hraw, const float* proj_w,
                      const float* proj_b, const float* v_w, const float* v_b, const float* out_w, const float* out_b,
                      const float* phase_in, const float* d_attn_out, float* d_x, float* d_hraw, float* d_proj_w,
                      float* d_proj_b, float* d_v_w, float* d_v_b, float* d_out_w, float* d_out_b);
}

using wave_hip::Rows;

namespace {

int g_failures = 0;

void assert_close(float got, float want, float tol, const std::string& label) {
  if (!(std::fabs(got - want) <= tol)) {
    std::printf("    %s: got %.9g want %.9g (tol %g)\n", label.c_str(), got, want, tol);
    throw std::runtime_error("assert_close failed: " + label);
  }
}

Rows rows_of(const std::vector<float>& flat, size_t T, size_t E) {
  Rows r(T, std::vector<float>(E));
  for (size_t t = 0; t < T; ++t)
    for (size_t e = 0; e < E; ++e) r[t][e] = flat[t * E + e];
  return r;
}

std::vector<float> flat_of(const Rows& r) {
  std::vector<float> f;
  for (const auto& row : r) f.insert(f.end(), row.begin(), row.end());
  return f;
}

// max-abs <= 1e-4 and relative L2 <= 1e-5 (the parity bar)
void assert_parity(const std::vector<float>& got, const std::vector<float>& want, const std::string& label) {
  double num = 0, den = 0, mx = 0;
  for (size_t i = 0; i < got.size(); ++i) {
    const double d = (double)got[i] - (double)want[i];
    num += d * d;
    den += (double)want[i] * want[i];
    mx = std::fmax(mx, std::fabs(d));
  }
  const double rel = den > 0 ? std::sqrt(num / den) : std::sqrt(num);
  std::printf("    %s: max_abs=%.3e rel_l2=%.3e\n", label.c_str(), mx, rel);
  if (!(mx <= 1e-4 && rel <= 1e-5)) throw std::runtime_error("parity failed: " + label);
}

struct Seq {
  size_t T, E, H;
  std::vector<float> q, k, v, d, att;
};

Seq make_seq(size_t T, size_t E, size_t H, uint64_t seed) {
  Seq s{T, E, H, {}, {}, {}, {}, {}};
  uint64_t st = seed;
  const double sd = 1.0 / std::sqrt((double)(E / H));
  for (auto* x : {&s.q, &s.k, &s.v}) {
    x->resize(T * E);
    wao_fill_normal(&st, x->data(), x->size(), sd);
  }
  s.d.resize(T * E);
  wao_fill_normal(&st, s.d.data(), s.d.size(), 1.0);
  s.att.resize(H * T * T);
  std::vector<float> out(T * E);
  wao_attention_core_fwd_f32(s.q.data(), s.k.data(), s.v.data(), (int)T, (int)E, (int)H, out.data(),
                             s.att.data(), nullptr);
  return s;
}

std::vector<Rows> att_rows(const Seq& s) {
  std::vector<Rows> a(s.H);
  for (size_t h = 0; h < s.H; ++h)
    a[h] = rows_of(std::vector<float>(s.att.begin() + h * s.T * s.T, s.att.begin() + (h + 1) * s.T * s.T),
                   s.T, s.T);
  return a;
}

void run(const char* name, const std::function<void()>& f) {
  try {
    f();
    std::printf("test %s ... ok\n", name);
  } catch (const std::exception& e) {
    std::printf("test %s ... FAILED (%s)\n", name, e.what());
    ++g_failures;
  }
  std::fflush(stdout);
}

// ---------------------------------------------------------------- tests

void test_softmax_backward_kat() {
  // src/common/math/attn_backward.rs:352-365 embedded in the full backward:
  // V = Q = K = I (D=2, one head) makes d_att = d_pre_proj = [[1,0],[2,4]].
  wave_hip::HipBackend be;
  Rows eye = {{1.f, 0.f}, {0.f, 1.f}};
  Rows d = {{1.f, 0.f}, {2.f, 4.f}};
  std::vector<Rows> att = {{{1.f, 0.f}, {0.3f, 0.7f}}};
  auto [dq, dk, dv] = be.attention_backward(d, eye, eye, eye, att, 1);
  const float scale = 1.0f / std::sqrt(2.0f);
  // d_score[0][0] = 0 -> dQ[0] = 0;  d_score[1] = [-0.42, 0.42] -> dQ[1] = scale * [-0.42, 0.42]
  assert_close(dq[0][0], 0.f, 1e-6f, "dq[0][0]");
  assert_close(dq[1][0], -0.42f * scale, 1e-4f, "dq[1][0]");
  assert_close(dq[1][1], 0.42f * scale, 1e-4f, "dq[1][1]");
  (void)dk;
  (void)dv;
}

void test_value_aggregation_backward_kat() {
  // src/common/math/attn_backward.rs:367-379: dV[0] = [1.0, 0.5]
  wave_hip::HipBackend be;
  Rows eye = {{1.f, 0.f}, {0.f, 1.f}};
  Rows v = {{1.f, 2.f}, {3.f, 4.f}};
  Rows d = {{1.f, 0.f}, {0.f, 1.f}};
  std::vector<Rows> att = {{{1.f, 0.f}, {0.5f, 0.5f}}};
  auto [dq, dk, dv] = be.attention_backward(d, eye, eye, v, att, 1);
  assert_close(dv[0][0], 1.0f, 1e-6f, "d_v[0][0]");
  assert_close(dv[0][1], 0.5f, 1e-6f, "d_v[0][1]");
  (void)dq;
  (void)dk;
}

void backward_vs_cpu(size_t T, size_t E, size_t H, uint64_t seed) {
  Seq s = make_seq(T, E, H, seed);
  wave_hip::HipBackend be;
  auto [dq, dk, dv] = be.attention_backward(rows_of(s.d, T, E), rows_of(s.q, T, E), rows_of(s.k, T, E),
                                            rows_of(s.v, T, E), att_rows(s), H);
  std::vector<float> rq(T * E), rk(T * E), rv(T * E);
  wao_attention_backward_f32(s.d.data(), s.q.data(), s.k.data(), s.v.data(), s.att.data(), (int)T, (int)E,
                             (int)H, rq.data(), rk.data(), rv.data());
  assert_parity(flat_of(dq), rq, "d_q");
  assert_parity(flat_of(dk), rk, "d_k");
  assert_parity(flat_of(dv), rv, "d_v");
}

void test_attention_backward_168_dim() { backward_vs_cpu(96, 168, 4, 42); }    // head_dim 42
void test_attention_backward_384_dim() { backward_vs_cpu(130, 384, 8, 7); }    // head_dim 48
void test_attention_backward_768_dim() { backward_vs_cpu(257, 768, 12, 3); }   // head_dim 64

void test_attention_core_matches_cpu() {
  for (auto cfg : {std::vector<size_t>{77, 168, 4}, std::vector<size_t>{200, 768, 12}}) {
    Seq s = make_seq(cfg[0], cfg[1], cfg[2], 99);
    wave_hip::HipBackend be;
    Rows o = be.attention_core(rows_of(s.q, s.T, s.E), rows_of(s.k, s.T, s.E), rows_of(s.v, s.T, s.E), s.H);
    std::vector<float> ref(s.T * s.E);
    wao_attention_core_fwd_f32(s.q.data(), s.k.data(), s.v.data(), (int)s.T, (int)s.E, (int)s.H, ref.data(),
                               nullptr, nullptr);
    assert_parity(flat_of(o), ref, "out");
  }
}

void test_attention_with_projections() {
  // ComputeBackend::attention(weights, x): c_attn, core, c_proj (src/common/compute.rs:357-414)
  for (auto cfg : {std::vector<size_t>{64, 168, 4}, std::vector<size_t>{150, 768, 12}}) {
    const size_t T = cfg[0], E = cfg[1], H = cfg[2];
    uint64_t st = 1234 + T;
    auto draw = [&](size_t n, double sd) {
      std::vector<float> v(n);
      wao_fill_normal(&st, v.data(), n, sd);
      return v;
    };
    const auto x = draw(T * E, 1.0), wa = draw(3 * E * E, 1.0 / std::sqrt((double)E)), ba = draw(3 * E, 0.1);
    const auto wp = draw(E * E, 1.0 / std::sqrt((double)E)), bp = draw(E, 0.1);
    wave_hip::AttentionWeights w{{rows_of(wa, 3 * E, E), ba}, {rows_of(wp, E, E), bp}, H};
    wave_hip::HipBackend be;
    Rows out = be.attention(w, rows_of(x, T, E));
    std::vector<float> ref(T * E);
    wao_attention_full_f32(x.data(), wa.data(), ba.data(), wp.data(), bp.data(), (int)T, (int)E, (int)H, ref.data());
    assert_parity(flat_of(out), ref, "attention out");
  }
}

void test_bad_head_count_panics() {
  wave_hip::HipBackend be;
  Rows x(4, std::vector<float>(10, 0.f));
  bool panicked = false;
  try {
    be.attention_core(x, x, x, 3);  // 10 % 3 != 0
  } catch (const wave_hip::Panic& p) {
    panicked = std::string(p.what()).find("divisible") != std::string::npos;
  }
  if (!panicked) throw std::runtime_error("expected a panic naming the divisibility rule");
}

void test_concurrent_callers() {
  // the reference calls the backend from one thread per batch element
  // (src/cpu/train_loop.rs:320-365); results must not depend on that
  const size_t T = 64, E = 192, H = 3;
  std::vector<Seq> seqs;
  for (int i = 0; i < 4; ++i) seqs.push_back(make_seq(T, E, H, 100 + i));
  std::vector<std::vector<float>> solo(4), conc(4);
  wave_hip::HipBackend be;
  for (int i = 0; i < 4; ++i) {
    auto r = be.attention_backward(rows_of(seqs[i].d, T, E), rows_of(seqs[i].q, T, E), rows_of(seqs[i].k, T, E),
                                   rows_of(seqs[i].v, T, E), att_rows(seqs[i]), H);
    solo[i] = flat_of(std::get<1>(r));
  }
  std::vector<std::thread> th;
  for (int i = 0; i < 4; ++i)
    th.emplace_back([&, i] {
      for (int rep = 0; rep < 3; ++rep) {
        auto r = be.attention_backward(rows_of(seqs[i].d, T, E), rows_of(seqs[i].q, T, E),
                                       rows_of(seqs[i].k, T, E), rows_of(seqs[i].v, T, E), att_rows(seqs[i]), H);
        conc[i] = flat_of(std::get<1>(r));
      }
    });
  for (auto& t : th) t.join();
  for (int i = 0; i < 4; ++i)
    if (solo[i] != conc[i]) throw std::runtime_error("concurrent result differs for sequence " + std::to_string(i));
}

// Wave attention through the C++ mirror (attn.rs:90-511) against the oracle,
// which replays the mirror's phases so both form the same bucket mask.
void wave_vs_cpu(size_t T, size_t E, size_t H, size_t C, uint64_t seed) {
  const size_t hd = E / H;
  uint64_t st = seed;
  auto normal = [&](size_t n, double sd) {
    std::vector<float> v(n);
    wao_fill_normal(&st, v.data(), n, sd);
    return v;
  };
  wave_hip::WaveAttnWeights w;
  for (size_t h = 0; h < H; ++h) {
    wave_hip::WaveAttnHeadWeights hw;
    hw.harmonic_raw = normal(1, 1.0)[0] + 0.5f;
    hw.phase_proj_w = rows_of(normal(2 * E, 1.0 / std::sqrt((double)E)), 2, E);
    hw.phase_proj_b = normal(2, 0.1);
    hw.v_proj_w = rows_of(normal(hd * hd, 1.0 / std::sqrt((double)hd)), hd, hd);
    hw.v_proj_b = normal(hd, 0.1);
    if (C) {
      hw.content_proj_w = rows_of(normal(C * E, 1.0 / std::sqrt((double)E)), C, E);
      hw.content_proj_b = normal(C, 0.1);
    }
    w.heads.push_back(hw);
  }
  w.out_proj_w = rows_of(normal(E * E, 1.0 / std::sqrt((double)E)), E, E);
  w.out_proj_b = normal(E, 0.1);
  const auto x = normal(T * E, 1.0);
  const auto dy = normal(T * E, 1.0 / std::sqrt((double)T));
  wave_hip::HipBackend be;
  Rows phases;
  const Rows out = be.wave_attention_forward(w, rows_of(x, T, E), E / 2, &phases);
  const auto ph = flat_of(phases);
  // oracle inputs in the packed layout
  const auto p = wave_hip::detail::pack_wave(w, E);
  std::vector<float> ref(T * E);
  wao_wave_fwd_f32(x.data(), (int)T, (int)E, (int)H, (int)C, p.hraw.data(), p.proj_w.data(), p.proj_b.data(),
                   p.v_w.data(), p.v_b.data(), p.out_w.data(), p.out_b.data(), ph.data(), ref.data(), nullptr,
                   nullptr, nullptr, nullptr, nullptr, nullptr, nullptr);
  assert_parity(flat_of(out), ref, "wave out");
  const auto g = be.wave_attention_backward_full(w, rows_of(x, T, E), rows_of(dy, T, E));
  const size_t P = 2 + C;
  std::vector<float> d_x(T * E), d_hraw(H), d_pw(H * P * E), d_pb(H * P), d_vw(H * hd * hd), d_vb(H * hd),
      d_ow(E * E), d_ob(E);
  wao_wave_bwd_f32(x.data(), (int)T, (int)E, (int)H, (int)C, p.hraw.data(), p.proj_w.data(), p.proj_b.data(),
                   p.v_w.data(), p.v_b.data(), p.out_w.data(), p.out_b.data(), ph.data(), dy.data(), d_x.data(),
                   d_hraw.data(), d_pw.data(), d_pb.data(), d_vw.data(), d_vb.data(), d_ow.data(), d_ob.data());
  assert_parity(flat_of(g.d_normed), d_x, "wave d_normed");
  assert_parity(flat_of(g.out_proj_w), d_ow, "wave d_out_proj_w");
  for (size_t h = 0; h < H; ++h) {
    assert_close(g.heads[h].d_harmonic_raw, d_hraw[h], 1e-4f, "d_harmonic_raw");
    std::vector<float> want_ph(d_pw.begin() + h * P * E, d_pw.begin() + h * P * E + 2 * E);
    assert_parity(flat_of(g.heads[h].phase_proj_w), want_ph, "d_phase_proj_w");
    std::vector<float> want_v(d_vw.begin() + h * hd * hd, d_vw.begin() + (h + 1) * hd * hd);
    assert_parity(flat_of(g.heads[h].v_proj_w), want_v, "d_v_proj_w");
    if (C) {
      std::vector<float> want_c(d_pw.begin() + h * P * E + 2 * E, d_pw.begin() + (h + 1) * P * E);
      assert_parity(flat_of(g.heads[h].content_proj_w), want_c, "d_content_proj_w");
    }
  }
  const Rows path = be.wave_attention_backward_pathway(w, rows_of(x, T, E), rows_of(dy, T, E));
  if (flat_of(path) != flat_of(g.d_normed)) throw std::runtime_error("pathway d_normed differs from the full backward");
}

void test_wave_attention_content() { wave_vs_cpu(130, 96, 4, 16, 77); }
void test_wave_attention_no_content() { wave_vs_cpu(65, 168, 4, 0, 78); }   // head_dim 42

}  // namespace

int main() {
  std::printf("wave_hip C++ host mirror tests (%s)\n", wha_version());
  run("softmax_backward_kat", test_softmax_backward_kat);
  run("value_aggregation_backward_kat", test_value_aggregation_backward_kat);
  run("attention_backward_168_dim", test_attention_backward_168_dim);
  run("attention_backward_384_dim", test_attention_backward_384_dim);
  run("attention_backward_768_dim", test_attention_backward_768_dim);
  run("attention_core_matches_cpu", test_attention_core_matches_cpu);
  run("attention_with_projections", test_attention_with_projections);
  run("bad_head_count_panics", test_bad_head_count_panics);
  run("concurrent_callers", test_concurrent_callers);
  run("wave_attention_content", test_wave_attention_content);
  run("wave_attention_no_content", test_wave_attention_no_content);
  std::printf("test result: %s. %d failed\n", g_failures ? "FAILED" : "ok", g_failures);
  return g_failures ? 1 : 0;
}
