/* wave_attn_oracle.c -- CPU restatement of wave-engine's dot-product causal
 * attention (forward core + backward), the seeded input generator, and a
 * threaded batch driver used as the CPU baseline.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product library (wave-engine_amd/) never links or calls it.
 *
 * Build: oracle/Makefile, gcc -O3 -ffp-contract=off, no fast-math, so every f32
 * sum is a sequential, non-contracted sum in the reference's loop order
 * (Rust never contracts a*b+c into an FMA).
 *
 * Followed reference code (paths relative to the reference checkout):
 *   src/common/compute.rs:357-414   attention_cpu (core :377-409)
 *   src/common/compute.rs:286-314   CpuBackend::attention_backward driver
 *   src/cpu/backward.rs:313-363     attention_backward_single
 *   src/common/math/attn_backward.rs:109-122  softmax_backward (same algebra)
 *   src/common/rng.rs:24-34         xorshift64 next_u64 / next_f32
 *   src/common/attn.rs:72-430       wave (harmonic coherence) attention forward
 *                                   and full backward (wave_core.inc)
 *   src/common/math/attn_backward.rs:13-323  its backward primitives
 * The Box-Muller normal draw is this build's own definition (the reference
 * has no normal sampler, src/common/rng.rs:5-45).
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ---- f32, reference order ---- */
#define REAL float
#define FN(name) name##_f32
#define EXPF expf
#define LOGF logf
#define SQRTF sqrtf
#define MAXF fmaxf
#define FABSF fabsf
#define ATAN2F atan2f
#define COSF cosf
#define SINF sinf
#define FMODF fmodf
#define WAVE_TAU 6.2831853071795864769f /* std::f32::consts::TAU */
#include "oracle_core.inc"
#include "wave_core.inc"
#undef FABSF
#undef ATAN2F
#undef COSF
#undef SINF
#undef FMODF
#undef WAVE_TAU
#undef REAL
#undef FN
#undef EXPF
#undef LOGF
#undef SQRTF
#undef MAXF

/* ---- f64 ground truth, same loops ---- */
#define REAL double
#define FN(name) name##_f64
#define EXPF exp
#define LOGF log
#define SQRTF sqrt
#define MAXF fmax
#define FABSF fabs
#define ATAN2F atan2
#define COSF cos
#define SINF sin
#define FMODF fmod
#define WAVE_TAU 6.2831853071795864769
#include "oracle_core.inc"
#include "wave_core.inc"
#undef FABSF
#undef ATAN2F
#undef COSF
#undef SINF
#undef FMODF
#undef WAVE_TAU
#undef REAL
#undef FN
#undef EXPF
#undef LOGF
#undef SQRTF
#undef MAXF

/* ---- generator ---- */

/* Rng::next_u64 (src/common/rng.rs:24-29). */
uint64_t wao_xorshift64_next(uint64_t* state) {
  uint64_t x = *state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *state = x;
  return x;
}

/* Rng::next_f32 (src/common/rng.rs:32-34): top 24 bits / 2^24, in [0,1). */
float wao_next_f32(uint64_t* state) {
  return (float)(wao_xorshift64_next(state) >> 40) / (float)(1u << 24);
}

/* Normal draws: each pair of uniforms (u1 = 1 - next_f32 in (0,1],
 * u2 = next_f32) gives r = sqrt(-2 ln u1), out[i] = r cos(2 pi u2) * stddev,
 * out[i+1] = r sin(2 pi u2) * stddev, evaluated in double and rounded once to
 * float.  An odd tail uses the cosine half and drops the sine half. */
void wao_fill_normal(uint64_t* state, float* out, size_t n, double stddev) {
  const double two_pi = 6.283185307179586476925286766559;
  size_t i = 0;
  while (i < n) {
    double u1 = 1.0 - (double)wao_next_f32(state);
    double u2 = (double)wao_next_f32(state);
    double r = sqrt(-2.0 * log(u1));
    out[i++] = (float)(r * cos(two_pi * u2) * stddev);
    if (i < n) out[i++] = (float)(r * sin(two_pi * u2) * stddev);
  }
}

/* ---- threaded batch driver (CPU baseline) ----
 * One thread per sequence, as the reference's training loop runs one scoped
 * thread per batch element (src/cpu/train_loop.rs:320-365).  Each sequence:
 * forward core producing att [H][T][T], then the backward from att. */
typedef struct {
  const float *q, *k, *v, *dout;
  float *out, *dq, *dk, *dv;
  int B, T, E, H, next_b, do_bwd;
  pthread_mutex_t mu;
} wao_job;

static void* wao_worker(void* arg) {
  wao_job* j = (wao_job*)arg;
  const size_t seq = (size_t)j->T * (size_t)j->E;
  float* att = NULL;
  if (j->do_bwd) att = (float*)malloc(sizeof(float) * (size_t)j->H * j->T * j->T);
  for (;;) {
    pthread_mutex_lock(&j->mu);
    int b = j->next_b++;
    pthread_mutex_unlock(&j->mu);
    if (b >= j->B) break;
    wao_attention_core_fwd_f32(j->q + b * seq, j->k + b * seq, j->v + b * seq,
                               j->T, j->E, j->H, j->out + b * seq, att, NULL);
    if (j->do_bwd)
      wao_attention_backward_f32(j->dout + b * seq, j->q + b * seq, j->k + b * seq,
                                 j->v + b * seq, att, j->T, j->E, j->H,
                                 j->dq + b * seq, j->dk + b * seq, j->dv + b * seq);
  }
  free(att);
  return NULL;
}

/* Runs B independent sequences ([B][T][E] each tensor) on nthreads threads.
 * dout/dq/dk/dv may be NULL for a forward-only run.  Returns 0. */
int wao_batch_fwd_bwd_f32(int B, int T, int E, int H, const float* q,
                          const float* k, const float* v, const float* dout,
                          float* out, float* dq, float* dk, float* dv,
                          int nthreads) {
  wao_job j;
  j.q = q; j.k = k; j.v = v; j.dout = dout;
  j.out = out; j.dq = dq; j.dk = dk; j.dv = dv;
  j.B = B; j.T = T; j.E = E; j.H = H; j.next_b = 0;
  j.do_bwd = (dout && dq && dk && dv) ? 1 : 0;
  pthread_mutex_init(&j.mu, NULL);
  if (nthreads < 1) nthreads = 1;
  if (nthreads > B) nthreads = B;
  pthread_t* th = (pthread_t*)malloc(sizeof(pthread_t) * (size_t)nthreads);
  for (int t = 0; t < nthreads; ++t) pthread_create(&th[t], NULL, wao_worker, &j);
  for (int t = 0; t < nthreads; ++t) pthread_join(th[t], NULL);
  free(th);
  pthread_mutex_destroy(&j.mu);
  return 0;
}
