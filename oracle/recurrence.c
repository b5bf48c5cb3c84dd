/*
 * fp64 brute-force gated delta rule, token by token -- TEST INFRASTRUCTURE ONLY.
 *
 * Pins the chunked oracle (oracle/gdn_ref.py chunk_rule) and, through it, the
 * HIP chunk kernel: the chunked form must equal this recurrence for any chunk
 * size, ragged length, initial state and head grouping.  Restates the
 * per-token update of nanovllm/models/qwen3_5.py:575-594 (and the upstream
 * T >= 1 loop it ports):
 *   q, k <- l2norm (eps 1e-6); q *= scale
 *   S <- S * exp(g);  delta = beta * (v - S^T k);  S <- S + k delta^T;  o = S^T q
 *
 * Layouts (row-major, one sequence):
 *   q, k [T, Hk, D]; v [T, Hv, D]; g, beta [T, Hv]; state [Hv, D, D];
 *   out [T, Hv, D].  Value head h reads key head h / (Hv / Hk).
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

void gdn_recurrence_f64(const double* q, const double* k, const double* v, const double* g,
                        const double* beta, double* state, double* out, int T, int Hk, int Hv,
                        int D, double scale, int l2norm) {
  double* qn = (double*)malloc(sizeof(double) * D);
  double* kn = (double*)malloc(sizeof(double) * D);
  double* kv = (double*)malloc(sizeof(double) * D);
  const int rep = Hv / Hk;
  for (int t = 0; t < T; ++t) {
    for (int h = 0; h < Hv; ++h) {
      const int kh = h / rep;
      const double* qp = q + ((size_t)t * Hk + kh) * D;
      const double* kp = k + ((size_t)t * Hk + kh) * D;
      const double* vp = v + ((size_t)t * Hv + h) * D;
      double qq = 0.0, kk = 0.0;
      for (int i = 0; i < D; ++i) {
        qq += qp[i] * qp[i];
        kk += kp[i] * kp[i];
      }
      const double rq = l2norm ? 1.0 / sqrt(qq + 1e-6) : 1.0;
      const double rk = l2norm ? 1.0 / sqrt(kk + 1e-6) : 1.0;
      for (int i = 0; i < D; ++i) {
        qn[i] = qp[i] * rq * scale;
        kn[i] = kp[i] * rk;
      }
      double* S = state + (size_t)h * D * D;
      const double decay = exp(g[(size_t)t * Hv + h]);
      const double b = beta[(size_t)t * Hv + h];
      for (int i = 0; i < D * D; ++i) S[i] *= decay;
      for (int j = 0; j < D; ++j) kv[j] = 0.0;
      for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j) kv[j] += S[(size_t)i * D + j] * kn[i];
      for (int j = 0; j < D; ++j) kv[j] = b * (vp[j] - kv[j]); /* delta */
      for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j) S[(size_t)i * D + j] += kn[i] * kv[j];
      double* op = out + ((size_t)t * Hv + h) * D;
      for (int j = 0; j < D; ++j) {
        double acc = 0.0;
        for (int i = 0; i < D; ++i) acc += S[(size_t)i * D + j] * qn[i];
        op[j] = acc;
      }
    }
  }
  free(qn);
  free(kn);
  free(kv);
}
