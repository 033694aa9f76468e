// hip_backend.hpp -- C++ host mirror of the attention half of wave-engine's
// ComputeBackend trait (reference src/common/compute.rs:8-174) and of the wave
// attention functions (src/common/attn.rs:90-511), built only on the C ABI of
// include/wave_hip_attn.h.  Header-only; link libwave_hip_attn.so.
//
// Same names, argument meaning and layouts as the reference:
//   Rows = Vec<Vec<f32>> ([T][n_embd], one row per position)
//   att_weights = [n_head][T][T] post-softmax rows
// and the reference's failure behaviour: its methods are infallible and panic
// (e.g. src/wgpu_tier/pipelines.rs:138, src/wgpu_tier/ops_forward.rs:63); here a
// failure throws wave_hip::Panic carrying the library's message.
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <stdexcept>
#include <string>
#include <tuple>
#include <vector>

#include "../../include/wave_hip_attn.h"

namespace wave_hip {

using Rows = std::vector<std::vector<float>>;

// LinearWeights (src/common/model.rs:175-180): w [out_dim][in_dim], b [out_dim].
struct LinearWeights {
  Rows w;
  std::vector<float> b;
};

// AttentionWeights (src/common/model.rs:189-195).
struct AttentionWeights {
  LinearWeights c_attn;  // [3*n_embd][n_embd]
  LinearWeights c_proj;  // [n_embd][n_embd]
  size_t n_head;
};

struct Panic : std::runtime_error {
  using std::runtime_error::runtime_error;
};

// WaveAttnHeadWeights / WaveAttnWeights (src/common/attn.rs:17-46): per head the
// harmonic number's raw parameter, the 2-row phase projection, the per-head value
// projection and the optional content projection (empty = none).
struct WaveAttnHeadWeights {
  float harmonic_raw = 0.f;
  Rows phase_proj_w;  // [2][n_embd]
  std::vector<float> phase_proj_b;  // [2]
  Rows v_proj_w;  // [head_dim][head_dim]
  std::vector<float> v_proj_b;  // [head_dim]
  Rows content_proj_w;  // [C][n_embd] or empty
  std::vector<float> content_proj_b;  // [C]
};

struct WaveAttnWeights {
  std::vector<WaveAttnHeadWeights> heads;
  Rows out_proj_w;  // [n_embd][n_embd]
  std::vector<float> out_proj_b;
};

// WaveAttnHeadGrads / WaveAttnGrads (attn.rs:317-336).
struct WaveAttnHeadGrads {
  Rows phase_proj_w;
  std::vector<float> phase_proj_b;
  Rows v_proj_w;
  std::vector<float> v_proj_b;
  Rows content_proj_w;
  std::vector<float> content_proj_b;
  float d_harmonic_raw = 0.f;
};

struct WaveAttnGrads {
  std::vector<WaveAttnHeadGrads> heads;
  Rows out_proj_w;
  std::vector<float> out_proj_b;
  Rows d_normed;
};

namespace detail {

inline void check(int rc, const char* what) {
  if (rc != WHA_OK) throw Panic(std::string(what) + " failed: " + wha_last_error());
}

inline std::vector<float> flatten(const Rows& rows, size_t T, size_t E, const char* name) {
  if (rows.size() != T) throw Panic(std::string(name) + ": expected " + std::to_string(T) + " rows");
  std::vector<float> flat(T * E);
  for (size_t t = 0; t < T; ++t) {
    if (rows[t].size() != E) throw Panic(std::string(name) + ": ragged row " + std::to_string(t));
    std::copy(rows[t].begin(), rows[t].end(), flat.begin() + t * E);
  }
  return flat;
}

inline Rows unflatten(const std::vector<float>& flat, size_t T, size_t E) {
  Rows r(T, std::vector<float>(E));
  for (size_t t = 0; t < T; ++t) std::copy(flat.begin() + t * E, flat.begin() + (t + 1) * E, r[t].begin());
  return r;
}

// Packs WaveAttnWeights into the ABI layout (host arrays): proj_w [H][2+C][E]
// with the phase rows first, then the content rows.
struct PackedWave {
  std::vector<float> hraw, proj_w, proj_b, v_w, v_b, out_w, out_b;
  size_t H = 0, C = 0, E = 0, hd = 0;
  wha_wave_weights view() const {
    return wha_wave_weights{hraw.data(), proj_w.data(), proj_b.data(), v_w.data(), v_b.data(), out_w.data(),
                            out_b.data()};
  }
};

inline PackedWave pack_wave(const WaveAttnWeights& w, size_t E) {
  PackedWave p;
  p.H = w.heads.size();
  if (p.H == 0) throw Panic("wave attention: no heads");
  p.C = w.heads[0].content_proj_w.size();
  p.E = E;
  p.hd = E / p.H;
  for (const auto& h : w.heads) {
    if (h.content_proj_w.size() != p.C) throw Panic("wave attention: heads differ in content_dim");
    p.hraw.push_back(h.harmonic_raw);
    const auto ph = flatten(h.phase_proj_w, 2, E, "phase_proj_w");
    p.proj_w.insert(p.proj_w.end(), ph.begin(), ph.end());
    if (p.C) {
      const auto cw = flatten(h.content_proj_w, p.C, E, "content_proj_w");
      p.proj_w.insert(p.proj_w.end(), cw.begin(), cw.end());
    }
    if (h.phase_proj_b.size() != 2 || h.content_proj_b.size() != p.C) throw Panic("wave attention: bias sizes");
    p.proj_b.insert(p.proj_b.end(), h.phase_proj_b.begin(), h.phase_proj_b.end());
    p.proj_b.insert(p.proj_b.end(), h.content_proj_b.begin(), h.content_proj_b.end());
    const auto vw = flatten(h.v_proj_w, p.hd, p.hd, "v_proj_w");
    p.v_w.insert(p.v_w.end(), vw.begin(), vw.end());
    if (h.v_proj_b.size() != p.hd) throw Panic("wave attention: v_proj_b size");
    p.v_b.insert(p.v_b.end(), h.v_proj_b.begin(), h.v_proj_b.end());
  }
  p.out_w = flatten(w.out_proj_w, E, E, "out_proj_w");
  if (w.out_proj_b.size() != E) throw Panic("wave attention: out_proj_b size");
  p.out_b = w.out_proj_b;
  return p;
}

}  // namespace detail

class HipBackend {
 public:
  // ComputeBackend::attention (src/common/compute.rs:42-43), i.e. attention_cpu
  // (:357-414) end to end: c_attn, causal attention core, c_proj.  x: [T][n_embd].
  Rows attention(const AttentionWeights& w, const Rows& x) const {
    const size_t T = x.size();
    if (T == 0) throw Panic("attention: empty sequence");
    const size_t E = x[0].size();
    if (w.c_attn.w.size() != 3 * E || w.c_attn.b.size() != 3 * E || w.c_proj.w.size() != E ||
        w.c_proj.b.size() != E)
      throw Panic("attention: c_attn must be [3E][E] + [3E] and c_proj [E][E] + [E]");
    const auto xf = detail::flatten(x, T, E, "x");
    const auto wa = detail::flatten(w.c_attn.w, 3 * E, E, "c_attn.w");
    const auto wp = detail::flatten(w.c_proj.w, E, E, "c_proj.w");
    std::vector<float> out(T * E);
    detail::check(wha_host_attention(xf.data(), wa.data(), w.c_attn.b.data(), wp.data(), w.c_proj.b.data(),
                                     (int32_t)T, (int32_t)E, (int32_t)w.n_head, out.data()),
                  "attention");
    return detail::unflatten(out, T, E);
  }

  // Core of attention_cpu (src/common/compute.rs:377-409): causal softmax
  // attention of already-projected q_all, k_all, v_all ([T][n_embd] each).
  Rows attention_core(const Rows& q_all, const Rows& k_all, const Rows& v_all, size_t n_head) const {
    const size_t T = q_all.size();
    if (T == 0) throw Panic("attention_core: empty sequence");
    const size_t E = q_all[0].size();
    const auto q = detail::flatten(q_all, T, E, "q_all");
    const auto k = detail::flatten(k_all, T, E, "k_all");
    const auto v = detail::flatten(v_all, T, E, "v_all");
    std::vector<float> o(T * E);
    detail::check(wha_host_attention_core_fwd(q.data(), k.data(), v.data(), (int32_t)T, (int32_t)E,
                                              (int32_t)n_head, o.data()),
                  "attention_core");
    return detail::unflatten(o, T, E);
  }

  // ComputeBackend::attention_backward (src/common/compute.rs:163-173) with
  // CpuBackend's semantics (:286-314): att_weights used as given.
  // Returns (d_q, d_k, d_v), each [T][n_embd].
  std::tuple<Rows, Rows, Rows> attention_backward(const Rows& d_pre_proj, const Rows& q_all,
                                                  const Rows& k_all, const Rows& v_all,
                                                  const std::vector<Rows>& att_weights,
                                                  size_t n_head) const {
    const size_t T = d_pre_proj.size();
    if (T == 0) throw Panic("attention_backward: empty sequence");
    const size_t E = d_pre_proj[0].size();
    const auto d = detail::flatten(d_pre_proj, T, E, "d_pre_proj");
    const auto q = detail::flatten(q_all, T, E, "q_all");
    const auto k = detail::flatten(k_all, T, E, "k_all");
    const auto v = detail::flatten(v_all, T, E, "v_all");
    if (att_weights.size() != n_head) throw Panic("attention_backward: att_weights must have n_head heads");
    std::vector<float> att(n_head * T * T);
    for (size_t h = 0; h < n_head; ++h) {
      const auto a = detail::flatten(att_weights[h], T, T, "att_weights[h]");
      std::copy(a.begin(), a.end(), att.begin() + h * T * T);
    }
    std::vector<float> dq(T * E), dk(T * E), dv(T * E);
    detail::check(wha_host_attention_backward(d.data(), q.data(), k.data(), v.data(), att.data(),
                                              (int32_t)T, (int32_t)E, (int32_t)n_head, dq.data(),
                                              dk.data(), dv.data()),
                  "attention_backward");
    return {detail::unflatten(dq, T, E), detail::unflatten(dk, T, E), detail::unflatten(dv, T, E)};
  }

  // wave_attention_forward (src/common/attn.rs:90-305) on one sequence of normed
  // hidden states x [T][n_embd], n_embd = 2 * n_bands.  Returns out (after
  // out_proj); phases (optional) receives [n_head][T] (WaveAttnCache.phases).
  // att_weights_all is not materialised; the device API recomputes rows on demand.
  Rows wave_attention_forward(const WaveAttnWeights& w, const Rows& x, size_t n_bands,
                              Rows* phases = nullptr) const {
    const size_t T = x.size();
    if (T == 0) throw Panic("wave_attention_forward: empty sequence");
    const size_t E = x[0].size();
    if (E != 2 * n_bands) throw Panic("wave_attention_forward: n_embd must be 2 * n_bands");
    const auto p = detail::pack_wave(w, E);
    const auto xf = detail::flatten(x, T, E, "x");
    std::vector<float> out(T * E), ph(p.H * T);
    const wha_wave_weights wv = p.view();
    detail::check(wha_host_wave_attention_forward(xf.data(), &wv, (int32_t)T, (int32_t)E, (int32_t)p.H,
                                                  (int32_t)p.C, out.data(), ph.data()),
                  "wave_attention_forward");
    if (phases) *phases = detail::unflatten(ph, p.H, T);
    return detail::unflatten(out, T, E);
  }

  // wave_attention_backward_full (attn.rs:346-430).  The reference passes the
  // forward's cache; here the forward is recomputed on the device from x.
  WaveAttnGrads wave_attention_backward_full(const WaveAttnWeights& w, const Rows& x, const Rows& d_attn_out) const {
    const size_t T = x.size();
    if (T == 0) throw Panic("wave_attention_backward_full: empty sequence");
    const size_t E = x[0].size();
    const auto p = detail::pack_wave(w, E);
    const auto xf = detail::flatten(x, T, E, "x");
    const auto df = detail::flatten(d_attn_out, T, E, "d_attn_out");
    const size_t P = 2 + p.C;
    std::vector<float> d_x(T * E), d_hraw(p.H), d_pw(p.H * P * E), d_pb(p.H * P), d_vw(p.H * p.hd * p.hd),
        d_vb(p.H * p.hd), d_ow(E * E), d_ob(E);
    const wha_wave_weights wv = p.view();
    const wha_wave_grads g{d_x.data(), d_hraw.data(), d_pw.data(), d_pb.data(), d_vw.data(), d_vb.data(),
                           d_ow.data(), d_ob.data()};
    detail::check(wha_host_wave_attention_backward(xf.data(), df.data(), &wv, (int32_t)T, (int32_t)E,
                                                   (int32_t)p.H, (int32_t)p.C, &g),
                  "wave_attention_backward_full");
    WaveAttnGrads out;
    for (size_t h = 0; h < p.H; ++h) {
      WaveAttnHeadGrads hg;
      const float* pw = d_pw.data() + h * P * E;
      hg.phase_proj_w = detail::unflatten(std::vector<float>(pw, pw + 2 * E), 2, E);
      hg.phase_proj_b = {d_pb[h * P], d_pb[h * P + 1]};
      if (p.C) {
        hg.content_proj_w = detail::unflatten(std::vector<float>(pw + 2 * E, pw + P * E), p.C, E);
        hg.content_proj_b.assign(d_pb.begin() + h * P + 2, d_pb.begin() + (h + 1) * P);
      }
      const float* vw = d_vw.data() + h * p.hd * p.hd;
      hg.v_proj_w = detail::unflatten(std::vector<float>(vw, vw + p.hd * p.hd), p.hd, p.hd);
      hg.v_proj_b.assign(d_vb.begin() + h * p.hd, d_vb.begin() + (h + 1) * p.hd);
      hg.d_harmonic_raw = d_hraw[h];
      out.heads.push_back(std::move(hg));
    }
    out.out_proj_w = detail::unflatten(d_ow, E, E);
    out.out_proj_b = d_ob;
    out.d_normed = detail::unflatten(d_x, T, E);
    return out;
  }

  // wave_attention_backward_pathway (attn.rs:432-511): d_normed only.
  Rows wave_attention_backward_pathway(const WaveAttnWeights& w, const Rows& x, const Rows& d_attn_out) const {
    const size_t T = x.size();
    if (T == 0) throw Panic("wave_attention_backward_pathway: empty sequence");
    const size_t E = x[0].size();
    const auto p = detail::pack_wave(w, E);
    const auto xf = detail::flatten(x, T, E, "x");
    const auto df = detail::flatten(d_attn_out, T, E, "d_attn_out");
    std::vector<float> d_x(T * E);
    const wha_wave_weights wv = p.view();
    const wha_wave_grads g{d_x.data(), nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr};
    detail::check(wha_host_wave_attention_backward(xf.data(), df.data(), &wv, (int32_t)T, (int32_t)E,
                                                   (int32_t)p.H, (int32_t)p.C, &g),
                  "wave_attention_backward_pathway");
    return detail::unflatten(d_x, T, E);
  }
};

}  // namespace wave_hip
