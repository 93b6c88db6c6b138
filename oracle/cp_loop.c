/*
 * Plain C restatement of the fixed-iteration Chambolle--Pock loop, for the CPU
 * baseline timing.
 *
 * TEST INFRASTRUCTURE ONLY: used by bench.py's cpu_baseline leg and by the
 * tests that pin it against the NumPy oracle (oracle/cp.py sparse_cp with
 * early_stop=False).  The product library never links or calls it.
 *
 * Follows the reference src/purin/solvers/chambolle_pock/kernels.py:
 *   cp_step 91-150       d+ = P(d + sigma (K ybar - r));
 *                        y+ = clip(a y - delta K^T d+ + delta yhat, lo, hi);
 *                        ybar+ = y+ + theta (y+ - y)
 *   prox 68-73           a = 1/(1 + tau q), delta = tau a, offset = -delta c
 *                        (q = 1, c = -yhat on the projection path)
 *   loop 228-290         y0 = yhat, ybar0 = y0, theta0 = 1; accelerated:
 *                        nt = 1/sqrt(1 + tau), tau <- nt tau, sigma <- sigma/nt,
 *                        theta <- nt (279-283)
 * with K given as a shared CSR of the kept, row-scaled rows.  The products use
 * the reference's accumulation orders: each row in slot order
 * (linalg/sparse/operators.py:518) and K^T v as a scatter over rows in
 * increasing order (operators.py:533).  max/clip propagate NaN like jnp.
 * Samples are independent; OpenMP splits them over threads.  Two instances:
 * purin_oracle_cp_fixed_f64 (double) and purin_oracle_cp_fixed_f32 (float,
 * every operation rounded to float like the reference's float32 runs).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define DEFINE_CP_LOOP(T, SUFFIX, SQRT)                                                        \
  static inline T max_nan_##SUFFIX(T x, T y) { return (x != x || x > y) ? x : y; }              \
  static inline T min_nan_##SUFFIX(T x, T y) { return (x != x || x < y) ? x : y; }              \
                                                                                               \
  static void one_sample_##SUFFIX(int64_t n, int64_t m, int64_t me, const int64_t* rptr,        \
                                  const int32_t* ridx, const T* rval, const T* r,               \
                                  const T* yhat, const T* lo, const T* hi, const T* d0,         \
                                  int64_t iterations, T tau, T sigma, int accelerated, T* y,    \
                                  T* d, T* ybar, T* t) {                                        \
    const T one = (T)1, zero = (T)0;                                                            \
    memcpy(y, yhat, (size_t)n * sizeof(T));                                                    \
    memcpy(ybar, yhat, (size_t)n * sizeof(T));                                                 \
    if (d0)                                                                                    \
      memcpy(d, d0, (size_t)m * sizeof(T));                                                    \
    else                                                                                       \
      memset(d, 0, (size_t)m * sizeof(T));                                                     \
    T theta = one;                                                                             \
    T a = one / (one + tau), delta = tau * a;                                                  \
    for (int64_t it = 0; it < iterations; ++it) {                                              \
      if (accelerated) {                                                                       \
        a = one / (one + tau);                                                                 \
        delta = tau * a;                                                                       \
      }                                                                                        \
      /* row pass: d+ = P(d + sigma (K ybar - r)), each row in slot order */                   \
      for (int64_t i = 0; i < m; ++i) {                                                        \
        T acc = zero;                                                                          \
        const int64_t b = rptr[i], e = rptr[i + 1];                                            \
        if (e > b) {                                                                           \
          acc = rval[b] * ybar[ridx[b]];                                                       \
          for (int64_t k = b + 1; k < e; ++k) acc = acc + rval[k] * ybar[ridx[k]];             \
        }                                                                                      \
        const T p = d[i] + sigma * (acc - r[i]);                                               \
        d[i] = i < me ? p : max_nan_##SUFFIX(p, zero);                                         \
      }                                                                                        \
      /* column pass: t = K^T d+ (scatter in row order), then the prox and clip */             \
      memset(t, 0, (size_t)n * sizeof(T));                                                     \
      for (int64_t i = 0; i < m; ++i)                                                          \
        for (int64_t k = rptr[i]; k < rptr[i + 1]; ++k)                                        \
          t[ridx[k]] = t[ridx[k]] + rval[k] * d[i];                                            \
      for (int64_t j = 0; j < n; ++j) {                                                        \
        const T pre = (a * y[j] - delta * t[j]) + delta * yhat[j];                             \
        const T yn = min_nan_##SUFFIX(max_nan_##SUFFIX(pre, lo[j]), hi[j]);                    \
        ybar[j] = yn + theta * (yn - y[j]);                                                    \
        y[j] = yn;                                                                             \
      }                                                                                        \
      if (accelerated) {                                                                       \
        const T nt = one / SQRT(one + tau);                                                    \
        tau = nt * tau;                                                                        \
        sigma = sigma / nt;                                                                    \
        theta = nt;                                                                            \
      }                                                                                        \
    }                                                                                          \
  }                                                                                            \
                                                                                               \
  int purin_oracle_cp_fixed_##SUFFIX(int64_t n, int64_t m, int64_t me, const int64_t* rptr,     \
                                     const int32_t* ridx, const T* rval, int64_t batch,         \
                                     const T* rhs, const T* target, const T* lower,             \
                                     const T* upper, const T* dual0, const T* tau,              \
                                     const T* sigma, int64_t iterations, int accelerated,       \
                                     int threads, T* y, T* d) {                                 \
    int failed = 0;                                                                            \
    _Pragma("omp parallel num_threads(threads > 0 ? threads : 1) reduction(| : failed)") {     \
      T* ybar = (T*)malloc((size_t)(n > 0 ? n : 1) * sizeof(T));                               \
      T* t = (T*)malloc((size_t)(n > 0 ? n : 1) * sizeof(T));                                  \
      const int ok = ybar && t;                                                                \
      if (!ok) failed = 1;                                                                     \
      /* every thread reaches the worksharing loop; one without scratch skips its samples */   \
      _Pragma("omp for schedule(static)") for (int64_t b = 0; b < batch; ++b) if (ok)          \
          one_sample_##SUFFIX(n, m, me, rptr, ridx, rval, rhs + b * m, target + b * n,         \
                              lower + b * n, upper + b * n, dual0 ? dual0 + b * m : NULL,      \
                              iterations, tau[b], sigma[b], accelerated, y + b * n, d + b * m, \
                              ybar, t);                                                        \
      free(ybar);                                                                              \
      free(t);                                                                                 \
    }                                                                                          \
    return failed;                                                                             \
  }

/*
 * batch samples, sample-major:
 *   rhs (batch, m) scaled kept right-hand sides; target (batch, n);
 *   lower, upper (batch, n); dual0 (batch, m) or NULL;
 *   tau, sigma (batch) initial steps.
 * Outputs y (batch, n), d (batch, m).  Returns 0, or 1 if scratch allocation fails.
 */
DEFINE_CP_LOOP(double, f64, sqrt)
DEFINE_CP_LOOP(float, f32, sqrtf)
