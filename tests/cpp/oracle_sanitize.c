/* Host AddressSanitizer / UndefinedBehaviorSanitizer run of the CPU oracle
 * (test infrastructure): every exported entry point, f32 and f64, at ragged
 * shapes, on heap buffers of exactly the documented sizes, so that an
 * out-of-bounds access, a use after free or undefined arithmetic in the
 * restatement is reported.  Built and run by tests/test_sanitizers.py
 * (tests/cpp/Makefile target `sanitize`); exit status 0 and no sanitizer
 * report means clean. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

/* prototypes of the oracle (oracle/wave_attn_oracle.c) */
#define DECL(REAL, S)                                                                                            \
  void wao_attention_core_fwd_##S(const REAL*, const REAL*, const REAL*, int, int, int, REAL*, REAL*, REAL*);   \
  void wao_attention_backward_##S(const REAL*, const REAL*, const REAL*, const REAL*, const REAL*, int, int, int, \
                                  REAL*, REAL*, REAL*);                                                          \
  void wao_decode_##S(const REAL*, const REAL*, const REAL*, int, int, int, REAL*, REAL*);                     \
  void wao_linear_##S(const REAL*, const REAL*, const REAL*, int, int, int, REAL*);                            \
  void wao_linear_backward_dx_##S(const REAL*, const REAL*, int, int, int, REAL*);                             \
  void wao_outer_product_accum_##S(const REAL*, const REAL*, int, int, int, REAL*, REAL*);                     \
  void wao_attention_full_##S(const REAL*, const REAL*, const REAL*, const REAL*, const REAL*, int, int, int,  \
                              REAL*);                                                                          \
  void wao_phases_##S(const REAL*, const REAL*, long, REAL*, int*);                                           \
  void wao_wave_fwd_##S(const REAL*, int, int, int, int, const REAL*, const REAL*, const REAL*, const REAL*,    \
                        const REAL*, const REAL*, const REAL*, const REAL*, REAL*, REAL*, REAL*, REAL*, REAL*,  \
                        REAL*, REAL*, REAL*);                                                                  \
  void wao_wave_bwd_##S(const REAL*, int, int, int, int, const REAL*, const REAL*, const REAL*, const REAL*,    \
                        const REAL*, const REAL*, const REAL*, const REAL*, const REAL*, REAL*, REAL*, REAL*,   \
                        REAL*, REAL*, REAL*, REAL*, REAL*);                                                    \
  void wao_wave_kv_prefill_##S(const REAL*, int, int, int, int, const REAL*, const REAL*, const REAL*,         \
                               const REAL*, const REAL*, const REAL*, const REAL*, const REAL*, REAL*, REAL*,  \
                               REAL*, REAL*);                                                                  \
  void wao_wave_kv_step_##S(const REAL*, int, int, int, const REAL*, const REAL*, const REAL*, const REAL*,     \
                            const REAL*, const REAL*, const REAL*, const REAL*, const REAL*, int, int,         \
                            const REAL*, REAL*, REAL*, REAL*, REAL*);
DECL(float, f32)
DECL(double, f64)
void wao_fill_normal(uint64_t* state, float* out, size_t n, double stddev);
int wao_batch_fwd_bwd_f32(int B, int T, int E, int H, const float* q, const float* k, const float* v,
                          const float* dout, float* out, float* dq, float* dk, float* dv, int nthreads);

static uint64_t g_state = 12345;

static float* randf(size_t n, double sd) {
  float* p = (float*)malloc(sizeof(float) * (n ? n : 1));
  wao_fill_normal(&g_state, p, n, sd);
  return p;
}
static double* randd(size_t n, double sd) {
  float* f = randf(n, sd);
  double* p = (double*)malloc(sizeof(double) * (n ? n : 1));
  for (size_t i = 0; i < n; ++i) p[i] = f[i];
  free(f);
  return p;
}

static int g_bad = 0;
static void check_finite_f(const char* what, const float* p, size_t n) {
  for (size_t i = 0; i < n; ++i)
    if (!isfinite(p[i])) {
      fprintf(stderr, "%s: non-finite at %zu\n", what, i);
      g_bad = 1;
      return;
    }
}

#define DOT_CASE(REAL, S, RAND)                                                                                  \
  static void dot_case_##S(int T, int E, int H) {                                                                \
    const size_t n = (size_t)T * E;                                                                              \
    REAL *q = RAND(n, 0.3), *k = RAND(n, 0.3), *v = RAND(n, 1.0), *d = RAND(n, 1.0);                          \
    REAL* o = (REAL*)malloc(sizeof(REAL) * n);                                                                   \
    REAL* att = (REAL*)malloc(sizeof(REAL) * (size_t)H * T * T);                                                 \
    REAL* lse = (REAL*)malloc(sizeof(REAL) * (size_t)H * T);                                                     \
    REAL *dq = (REAL*)malloc(sizeof(REAL) * n), *dk = (REAL*)malloc(sizeof(REAL) * n),                           \
         *dv = (REAL*)malloc(sizeof(REAL) * n);                                                                  \
    wao_attention_core_fwd_##S(q, k, v, T, E, H, o, att, lse);                                                  \
    wao_attention_core_fwd_##S(q, k, v, T, E, H, o, NULL, NULL);                                                \
    wao_attention_backward_##S(d, q, k, v, att, T, E, H, dq, dk, dv);                                           \
    REAL* od = (REAL*)malloc(sizeof(REAL) * E);                                                                  \
    REAL* ld = (REAL*)malloc(sizeof(REAL) * H);                                                                  \
    wao_decode_##S(q + (size_t)(T - 1) * E, k, v, T, E, H, od, ld);                                             \
    free(q); free(k); free(v); free(d); free(o); free(att); free(lse); free(dq); free(dk); free(dv);            \
    free(od); free(ld);                                                                                          \
  }
DOT_CASE(float, f32, randf)
DOT_CASE(double, f64, randd)

#define LIN_CASE(REAL, S, RAND)                                                                                  \
  static void lin_case_##S(int M, int N, int K) {                                                                \
    REAL *x = RAND((size_t)M * K, 1.0), *w = RAND((size_t)N * K, 0.1), *b = RAND(N, 0.1);                     \
    REAL *y = (REAL*)malloc(sizeof(REAL) * M * N), *dx = (REAL*)malloc(sizeof(REAL) * M * K);                   \
    REAL *dw = (REAL*)malloc(sizeof(REAL) * N * K), *db = (REAL*)malloc(sizeof(REAL) * N);                      \
    wao_linear_##S(x, w, b, M, N, K, y);                                                                        \
    wao_linear_##S(x, w, NULL, M, N, K, y);                                                                     \
    wao_linear_backward_dx_##S(y, w, M, N, K, dx);                                                              \
    wao_outer_product_accum_##S(y, x, M, N, K, dw, db);                                                        \
    wao_outer_product_accum_##S(y, x, M, N, K, dw, NULL);                                                      \
    free(x); free(w); free(b); free(y); free(dx); free(dw); free(db);                                          \
  }
LIN_CASE(float, f32, randf)
LIN_CASE(double, f64, randd)

#define FULL_CASE(REAL, S, RAND)                                                                                 \
  static void full_case_##S(int T, int E, int H) {                                                               \
    REAL *x = RAND((size_t)T * E, 1.0), *wa = RAND((size_t)3 * E * E, 0.05), *ba = RAND(3 * E, 0.1);          \
    REAL *wp = RAND((size_t)E * E, 0.05), *bp = RAND(E, 0.1), *o = (REAL*)malloc(sizeof(REAL) * T * E);        \
    wao_attention_full_##S(x, wa, ba, wp, bp, T, E, H, o);                                                     \
    free(x); free(wa); free(ba); free(wp); free(bp); free(o);                                                   \
  }
FULL_CASE(float, f32, randf)
FULL_CASE(double, f64, randd)

#define WAVE_CASE(REAL, S, RAND)                                                                                 \
  static void wave_case_##S(int T, int E, int H, int C) {                                                        \
    const int hd = E / H, P = 2 + C;                                                                             \
    REAL *x = RAND((size_t)T * E, 1.0), *hr = RAND(H, 1.0), *pw = RAND((size_t)H * P * E, 0.1);              \
    REAL *pb = RAND((size_t)H * P, 0.1), *vw = RAND((size_t)H * hd * hd, 0.2), *vb = RAND((size_t)H * hd, 0.1);\
    REAL *ow = RAND((size_t)E * E, 0.1), *ob = RAND(E, 0.1), *dy = RAND((size_t)T * E, 1.0);                  \
    REAL* out = (REAL*)malloc(sizeof(REAL) * T * E);                                                             \
    REAL* merged = (REAL*)malloc(sizeof(REAL) * T * E);                                                          \
    REAL* att = (REAL*)malloc(sizeof(REAL) * (size_t)H * T * T);                                                 \
    REAL* ph = (REAL*)malloc(sizeof(REAL) * H * T);                                                              \
    REAL* rs = (REAL*)malloc(sizeof(REAL) * H * T * 2);                                                          \
    REAL* cv = C > 0 ? (REAL*)malloc(sizeof(REAL) * H * T * C) : NULL;                                           \
    REAL* vals = (REAL*)malloc(sizeof(REAL) * (size_t)H * T * hd);                                               \
    REAL* lse = (REAL*)malloc(sizeof(REAL) * H * T);                                                             \
    wao_wave_fwd_##S(x, T, E, H, C, hr, pw, pb, vw, vb, ow, ob, NULL, out, merged, att, ph, rs, cv, vals, lse);  \
    wao_wave_fwd_##S(x, T, E, H, C, hr, pw, pb, vw, vb, ow, ob, ph, out, NULL, NULL, NULL, NULL, NULL, NULL,     \
                     NULL);                                                                                      \
    REAL *dx = (REAL*)malloc(sizeof(REAL) * T * E), *dh = (REAL*)malloc(sizeof(REAL) * H);                      \
    REAL *dpw = (REAL*)malloc(sizeof(REAL) * H * P * E), *dpb = (REAL*)malloc(sizeof(REAL) * H * P);            \
    REAL *dvw = (REAL*)malloc(sizeof(REAL) * H * hd * hd), *dvb = (REAL*)malloc(sizeof(REAL) * H * hd);         \
    REAL *dow = (REAL*)malloc(sizeof(REAL) * E * E), *dob = (REAL*)malloc(sizeof(REAL) * E);                    \
    wao_wave_bwd_##S(x, T, E, H, C, hr, pw, pb, vw, vb, ow, ob, NULL, dy, dx, dh, dpw, dpb, dvw, dvb, dow, dob); \
    REAL* kph = (REAL*)malloc(sizeof(REAL) * H * T);                                                             \
    REAL* kvals = (REAL*)malloc(sizeof(REAL) * (size_t)H * T * hd);                                              \
    wao_wave_kv_prefill_##S(x, T, E, H, C, hr, pw, pb, vw, vb, ow, ob, NULL, out, kph, kvals, merged);          \
    REAL *o1 = (REAL*)malloc(sizeof(REAL) * E), *pn = (REAL*)malloc(sizeof(REAL) * H);                           \
    REAL *vn = (REAL*)malloc(sizeof(REAL) * H * hd), *m1 = (REAL*)malloc(sizeof(REAL) * E);                      \
    wao_wave_kv_step_##S(x + (size_t)(T - 1) * E, E, H, C, hr, pw, pb, vw, vb, ow, ob, kph, kvals, T, T - 1,    \
                         NULL, o1, pn, vn, m1);                                                                  \
    REAL* phs = (REAL*)malloc(sizeof(REAL) * H * T);                                                             \
    int* bks = (int*)malloc(sizeof(int) * H * T);                                                                \
    wao_phases_##S(rs, rs + H * T, (long)H * T, phs, bks);                                                       \
    free(x); free(hr); free(pw); free(pb); free(vw); free(vb); free(ow); free(ob); free(dy); free(out);        \
    free(merged); free(att); free(ph); free(rs); free(cv); free(vals); free(lse); free(dx); free(dh);           \
    free(dpw); free(dpb); free(dvw); free(dvb); free(dow); free(dob); free(kph); free(kvals); free(o1);         \
    free(pn); free(vn); free(m1); free(phs); free(bks);                                                         \
  }
WAVE_CASE(float, f32, randf)
WAVE_CASE(double, f64, randd)

int main(void) {
  static const int dot[][3] = {{1, 8, 1}, {17, 16, 2}, {65, 84, 2}, {100, 192, 3}, {130, 128, 1}, {33, 84, 1}};
  for (size_t i = 0; i < sizeof(dot) / sizeof(dot[0]); ++i) {
    dot_case_f32(dot[i][0], dot[i][1], dot[i][2]);
    dot_case_f64(dot[i][0], dot[i][1], dot[i][2]);
  }
  static const int lin[][3] = {{1, 1, 1}, {7, 13, 5}, {33, 24, 40}};
  for (size_t i = 0; i < sizeof(lin) / sizeof(lin[0]); ++i) {
    lin_case_f32(lin[i][0], lin[i][1], lin[i][2]);
    lin_case_f64(lin[i][0], lin[i][1], lin[i][2]);
  }
  full_case_f32(19, 24, 3);
  full_case_f64(19, 24, 3);
  static const int wav[][4] = {{1, 16, 2, 0}, {9, 24, 2, 5}, {40, 48, 4, 16}, {33, 12, 1, 30}};
  for (size_t i = 0; i < sizeof(wav) / sizeof(wav[0]); ++i) {
    wave_case_f32(wav[i][0], wav[i][1], wav[i][2], wav[i][3]);
    wave_case_f64(wav[i][0], wav[i][1], wav[i][2], wav[i][3]);
  }
  /* the threaded batch driver (the CPU baseline), 3 sequences on 2 threads */
  const int B = 3, T = 37, E = 48, H = 3;
  const size_t n = (size_t)B * T * E;
  float *q = randf(n, 0.3), *k = randf(n, 0.3), *v = randf(n, 1.0), *d = randf(n, 1.0);
  float *o = (float*)malloc(sizeof(float) * n), *dq = (float*)malloc(sizeof(float) * n);
  float *dk = (float*)malloc(sizeof(float) * n), *dv = (float*)malloc(sizeof(float) * n);
  if (wao_batch_fwd_bwd_f32(B, T, E, H, q, k, v, d, o, dq, dk, dv, 2) != 0) g_bad = 1;
  check_finite_f("batch out", o, n);
  check_finite_f("batch dq", dq, n);
  free(q); free(k); free(v); free(d); free(o); free(dq); free(dk); free(dv);
  printf(g_bad ? "oracle_sanitize: FAILED\n" : "oracle_sanitize: OK\n");
  return g_bad;
}
