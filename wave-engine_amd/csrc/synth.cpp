// Seeded synthetic inputs for benchmarks and tests (host code).
//
// Stream definition: xorshift64 exactly as the reference's Rng::next_u64 /
// next_f32 (src/common/rng.rs:24-34); normals by Box-Muller on consecutive
// pairs of uniforms (u1 = 1 - next_f32 in (0,1], u2 = next_f32),
// out[2i] = r cos(2 pi u2), out[2i+1] = r sin(2 pi u2), r = sqrt(-2 ln u1),
// evaluated in double, times stddev, rounded once to float.
//
// The generator is linear over GF(2): one step is a 64x64 bit matrix M, so
// the state after n steps is M^n s.  Large requests are split into segments
// whose start states are obtained by jumping ahead with M^(offset), and the
// segments are filled on several threads.  The output is bit-identical to the
// sequential stream.
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

inline uint64_t step(uint64_t x) {
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  return x;
}

inline float to_unit(uint64_t x) { return (float)(x >> 40) / (float)(1u << 24); }

// 64x64 GF(2) matrix as 64 column images: col[j] = M e_j.
struct Mat {
  uint64_t col[64];
};

inline uint64_t apply(const Mat& m, uint64_t v) {
  uint64_t r = 0;
  for (int j = 0; j < 64; ++j)
    if ((v >> j) & 1u) r ^= m.col[j];
  return r;
}

Mat mul(const Mat& a, const Mat& b) {  // a*b
  Mat r;
  for (int j = 0; j < 64; ++j) r.col[j] = apply(a, b.col[j]);
  return r;
}

Mat step_matrix() {
  Mat m;
  for (int j = 0; j < 64; ++j) m.col[j] = step(uint64_t(1) << j);
  return m;
}

uint64_t jump(uint64_t state, uint64_t n) {
  Mat p = step_matrix();
  while (n) {
    if (n & 1u) state = apply(p, state);
    p = mul(p, p);
    n >>= 1;
  }
  return state;
}

void fill_pairs(uint64_t state, float* out, size_t n, double stddev) {
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    state = step(state);
    const double u1 = 1.0 - (double)to_unit(state);
    state = step(state);
    const double u2 = (double)to_unit(state);
    const double r = std::sqrt(-2.0 * std::log(u1));
    out[i++] = (float)(r * std::cos(two_pi * u2) * stddev);
    if (i < n) out[i++] = (float)(r * std::sin(two_pi * u2) * stddev);
  }
}

}  // namespace

extern "C" {

// Fills out[0..n) with normal draws continuing the stream in *state and
// advances *state by 2*ceil(n/2) steps.  nthreads <= 0 picks a default.
// Returns 0, or -1 for a zero state (xorshift64 is stuck at zero).
int wha_synth_normal(uint64_t* state, float* out, size_t n, double stddev, int nthreads) {
  if (state == nullptr || *state == 0) return -1;
  const size_t npairs = (n + 1) / 2;
  const uint64_t s0 = *state;
  const size_t kMinPerThread = size_t(1) << 20;
  int nt = nthreads > 0 ? nthreads : (int)std::thread::hardware_concurrency();
  if (nt > 16) nt = 16;
  if (nt < 1) nt = 1;
  if ((size_t)nt > npairs / (kMinPerThread / 2) + 1) nt = (int)(npairs / (kMinPerThread / 2) + 1);
  if (nt <= 1) {
    fill_pairs(s0, out, n, stddev);
  } else {
    const size_t per = (npairs + nt - 1) / nt;  // pairs per segment
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
      const size_t p0 = (size_t)t * per;
      if (p0 >= npairs) break;
      const size_t p1 = p0 + per < npairs ? p0 + per : npairs;
      const size_t e0 = 2 * p0;
      const size_t e1 = (2 * p1 < n) ? 2 * p1 : n;
      th.emplace_back([=] { fill_pairs(jump(s0, 2 * (uint64_t)p0), out + e0, e1 - e0, stddev); });
    }
    for (auto& x : th) x.join();
  }
  *state = jump(s0, 2 * (uint64_t)npairs);
  return 0;
}

}  // extern "C"
