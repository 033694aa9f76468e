// hip_backend.hpp -- C++ host mirror of the attention half of wave-engine's
// ComputeBackend trait (reference src/common/compute.rs:8-174), built only on
// the C ABI of include/wave_hip_attn.h.  Header-only; link libwave_hip_attn.so.
//
// Same names, argument meaning and layouts as the reference:
//   Rows = Vec<Vec<f32>> ([T][n_embd], one row per position)
//   att_weights = [n_head][T][T] post-softmax rows
// and the reference's failure behaviour: its methods are infallible and panic
// (e.g. src/wgpu_tier/pipelines.rs:138, src/wgpu_tier/ops_forward.rs:63); here a
// failure throws wave_hip::Panic carrying the library's message.
#pragma once

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
};

}  // namespace wave_hip
