/*
 * CPU oracle for the Avey / Avey-B forward contextualizer (plain C, fp64).
 *
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (ctypes) to cross-check the numpy
 * oracle in oracle/avey_oracle.py. The product library never links this file.
 *
 * It restates the reference's eager algorithm (avey_kernels/ops.py:61-91) in a
 * different order from the numpy restatement: one query row at a time,
 * streaming over keys, never forming the C x C similarity matrix. Agreement of
 * the two restatements on random inputs pins the numpy oracle against slips
 * that a single formulation would hide (a transposed V, a wrong mask edge, a
 * denominator taken after the bias, ...).
 *
 * Accumulation is in long double; inputs and outputs are double.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>

enum { ACT_IDENTITY = 0, ACT_RELU = 1, ACT_RELU2 = 2, ACT_SILU = 3, ACT_GELU = 4 };

/* ops.py:49-58 */
static long double activate(long double x, int act) {
  switch (act) {
    case ACT_RELU: return x > 0 ? x : 0;
    case ACT_RELU2: return x > 0 ? x * x : 0;
    case ACT_SILU: return x / (1.0L + expl(-x));
    case ACT_GELU: {
      const long double k = sqrtl(2.0L / 3.14159265358979323846264338327950288L);
      return 0.5L * x * (1.0L + tanhl(k * (x + 0.044715L * x * x * x)));
    }
    default: return x;
  }
}

/*
 * z_tr, z_tl, out: [B][C][D] row-major; v: [C][C] (query, key) or NULL;
 * z_tl, bias, valid may be NULL. Returns 0, or -1 on allocation failure.
 */
int avey_oracle_f64(const double* z_tr, const double* v, const double* z_tl, const double* bias,
                    const uint8_t* valid, double* out, int64_t B, int64_t C, int64_t D, int causal,
                    int normalize, int act, double eps, double norm_eps) {
  long double* inv = (long double*)malloc(sizeof(long double) * (size_t)C);
  long double* num = (long double*)malloc(sizeof(long double) * (size_t)D);
  if (!inv || !num) {
    free(inv);
    free(num);
    return -1;
  }
  for (int64_t b = 0; b < B; ++b) {
    const double* zb = z_tr + b * C * D;
    const uint8_t* vb = valid ? valid + b * C : NULL;
    /* ops.py:64-68: padded rows count as zero rows; F.normalize clamps the norm. */
    for (int64_t j = 0; j < C; ++j) {
      long double ss = 0;
      if (!vb || vb[j])
        for (int64_t f = 0; f < D; ++f) ss += (long double)zb[j * D + f] * zb[j * D + f];
      long double n = sqrtl(ss);
      inv[j] = 1.0L / (n > norm_eps ? n : (long double)norm_eps);
    }
    for (int64_t i = 0; i < C; ++i) {
      double* ob = out + (b * C + i) * D;
      const int row_ok = !vb || vb[i];
      for (int64_t f = 0; f < D; ++f) num[f] = 0;
      long double den = 0;
      const int64_t last = causal ? i : C - 1; /* ops.py:72-75: keep j <= i */
      for (int64_t j = 0; j <= last && row_ok; ++j) {
        if (vb && !vb[j]) continue; /* ops.py:76-77 */
        long double dot = 0;
        for (int64_t f = 0; f < D; ++f) dot += (long double)zb[i * D + f] * zb[j * D + f];
        long double s = dot * inv[i] * inv[j];         /* ops.py:68-69 */
        if (v) s *= (long double)v[i * C + j];          /* ops.py:70-71 */
        den += s;
        for (int64_t f = 0; f < D; ++f) num[f] += s * zb[j * D + f]; /* ops.py:78 */
      }
      for (int64_t f = 0; f < D; ++f) {
        if (!row_ok) { /* ops.py:89-90 */
          ob[f] = 0.0;
          continue;
        }
        long double y = num[f];
        if (normalize) y = y / (den + (long double)eps); /* ops.py:79-80 */
        if (bias) y += bias[f];                          /* ops.py:81-82 */
        y = activate(y, act);                            /* ops.py:83 */
        if (z_tl) y *= (long double)z_tl[(b * C + i) * D + f]; /* ops.py:84-88 */
        ob[f] = (double)y;
      }
    }
  }
  free(inv);
  free(num);
  return 0;
}
