/*
 * flce_ref.c -- TEST INFRASTRUCTURE ONLY.  Plain-C restatement of the fused
 * LM-head linear + per-token cross-entropy algorithm, used to check the HIP
 * library on the CPU side of the tests.  Never linked into the product.
 *
 * Algorithm followed (the reference reaches it at none_reduction_losses.py:16-23):
 *   LIGER:ops/fused_linear_cross_entropy.py::fused_linear_cross_entropy_forward
 *     - count of non-ignored targets (target != ignore_index)   -> ref_prepare
 *     - per row chunk: logits = X_c W^T in the model dtype        -> ref_forward
 *   LIGER:ops/cross_entropy.py::liger_cross_entropy_kernel
 *     - online max / sum-exp over the row in blocks -> lse,
 *       loss = lse - x_y, 0 for ignored rows; grad = softmax - onehot
 *   LIGER:ops/fused_linear_cross_entropy.py (chunk GEMMs)
 *     - dX = G W, dW += G^T X                                     -> ref_backward
 * with the per-token upstream gradient of train.py:98-104 and the torch-path
 * semantics of none_reduction_losses.py:35 (logits rounded to the model dtype
 * as F.linear returns them, then evaluated in fp32/fp64).
 * The per-sample sums (ref_segment_sum) follow the packed layout of
 * sampler.py:182-188.  ref_ce_forward is F.cross_entropy(reduction='none')
 * over materialised logits (none_reduction_losses.py:35).
 *
 * Accumulation is in double.  Pinned in tests/test_oracle.py against the
 * float64 closed forms of oracle/brute.py, the torch path, and invariants.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* Round a float to the nearest bfloat16 (ties to even), returned as float. */
static float round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) { /* inf / nan unchanged */
    u &= 0xffff0000u;
    if (x != x) u |= 0x00400000u;
  } else {
    u += 0x7fffu + ((u >> 16) & 1u);
    u &= 0xffff0000u;
  }
  memcpy(&x, &u, 4);
  return x;
}

float ref_round_bf16(float x) { return round_bf16(x); }

/* Valid rows first (ascending t), then every other row from the end of
 * row_index backwards; counts = {N, #bad labels, first bad t or -1, 0}. */
int ref_prepare(const int64_t* labels, int64_t T, int64_t V, int64_t ignore, int shift,
                int32_t* row_index, int32_t* row_label, int32_t* counts) {
  int64_t nv = 0, nm = 0, bad = 0, first_bad = -1;
  for (int64_t t = 0; t < T; ++t) {
    int64_t lab = shift ? (t + 1 < T ? labels[t + 1] : ignore) : labels[t];
    if (lab != ignore && lab >= 0 && lab < V) {
      row_index[nv] = (int32_t)t;
      row_label[nv] = (int32_t)lab;
      ++nv;
    } else {
      if (lab != ignore) {
        if (first_bad < 0) first_bad = t;
        ++bad;
      }
      row_index[T - 1 - nm] = (int32_t)t;
      ++nm;
    }
  }
  counts[0] = (int32_t)nv;
  counts[1] = (int32_t)bad;
  counts[2] = (int32_t)first_bad;
  counts[3] = 0;
  return 0;
}

static double logit(const float* X, const float* W, int64_t H, int64_t t, int64_t v,
                    int round_bf, double cap, double* dcap) {
  double s = 0.0;
  for (int64_t h = 0; h < H; ++h) s += (double)X[t * H + h] * (double)W[v * H + h];
  float sf = (float)s;
  if (round_bf) sf = round_bf16(sf);
  double z = sf;
  *dcap = 1.0;
  if (cap > 0.0) {
    double th = tanh(z / cap);
    z = cap * th;
    *dcap = 1.0 - th * th;
  }
  return z;
}

/* Online log-sum-exp over blocks of 256 columns (one block = one update of
 * the running (max, sum) pair). */
void ref_forward(const float* X, const float* W, int64_t T, int64_t H, int64_t V, int round_bf,
                 double cap, const int32_t* row_index, const int32_t* row_label, int64_t N,
                 float* loss, float* lse) {
  for (int64_t t = 0; t < T; ++t) loss[t] = 0.0f;
  for (int64_t i = 0; i < N; ++i) {
    const int64_t t = row_index[i], y = row_label[i];
    double m = -INFINITY, d = 0.0, xy = 0.0, dc;
    for (int64_t v0 = 0; v0 < V; v0 += 256) {
      const int64_t v1 = v0 + 256 < V ? v0 + 256 : V;
      double bm = -INFINITY;
      double z[256];
      for (int64_t v = v0; v < v1; ++v) {
        z[v - v0] = logit(X, W, H, t, v, round_bf, cap, &dc);
        if (z[v - v0] > bm) bm = z[v - v0];
        if (v == y) xy = z[v - v0];
      }
      const double mn = bm > m ? bm : m;
      double s = 0.0;
      for (int64_t v = v0; v < v1; ++v) s += exp(z[v - v0] - mn);
      d = d * exp(m - mn) + s;
      m = mn;
    }
    const double L = m + log(d);
    lse[i] = (float)L;
    loss[t] = (float)(L - xy);
  }
}

/* dX [T, H] (rows of ignored tokens zeroed), dW [V, H] (+)= G^T X.
 * G = g_t (exp(z - lse) - onehot) * softcap', rounded to bf16 when round_bf
 * (the model-dtype cast of the logits gradient); dX is rounded likewise. */
void ref_backward(const float* X, const float* W, int64_t T, int64_t H, int64_t V, int round_bf,
                  double cap, const int32_t* row_index, const int32_t* row_label, int64_t N,
                  const float* lse, const float* grad, int64_t gstride, float* dX, float* dW,
                  int accumulate) {
  double* dWd = (double*)malloc(sizeof(double) * (size_t)(V * H));
  double* acc = (double*)malloc(sizeof(double) * (size_t)H);
  for (int64_t k = 0; k < V * H; ++k) dWd[k] = accumulate ? (double)dW[k] : 0.0;
  for (int64_t k = 0; k < T * H; ++k) dX[k] = 0.0f;
  for (int64_t i = 0; i < N; ++i) {
    const int64_t t = row_index[i], y = row_label[i];
    const double g = grad[t * gstride];
    for (int64_t h = 0; h < H; ++h) acc[h] = 0.0;
    for (int64_t v = 0; v < V; ++v) {
      double dc;
      const double z = logit(X, W, H, t, v, round_bf, cap, &dc);
      double G = g * (exp(z - (double)lse[i]) - (v == y ? 1.0 : 0.0)) * dc;
      float Gf = (float)G;
      if (round_bf) Gf = round_bf16(Gf);
      for (int64_t h = 0; h < H; ++h) {
        acc[h] += (double)Gf * (double)W[v * H + h];
        dWd[v * H + h] += (double)Gf * (double)X[t * H + h];
      }
    }
    for (int64_t h = 0; h < H; ++h) {
      float o = (float)acc[h];
      dX[t * H + h] = round_bf ? round_bf16(o) : o;
    }
  }
  for (int64_t k = 0; k < V * H; ++k) dW[k] = (float)dWd[k];
  free(acc);
  free(dWd);
}

void ref_segment_sum(const float* loss, const int64_t* target, int64_t T, int64_t ignore,
                     const int32_t* cu, int64_t S, float* seg_loss, int32_t* seg_count,
                     int32_t* status) {
  int bad = (cu[0] != 0 || (int64_t)cu[S] != T);
  for (int64_t s = 0; s < S; ++s)
    if (cu[s + 1] < cu[s]) bad = 1;
  *status = bad;
  for (int64_t s = 0; s < S; ++s) {
    double a = 0.0;
    int32_t c = 0;
    if (!bad)
      for (int64_t t = cu[s]; t < cu[s + 1]; ++t) {
        a += loss[t];
        c += target[t] != ignore;
      }
    seg_loss[s] = (float)a;
    seg_count[s] = c;
  }
}

void ref_ce_forward(const float* logits, int64_t T, int64_t V, const int64_t* target,
                    int64_t ignore, float* loss, float* lse, int32_t* status) {
  *status = 0;
  for (int64_t t = 0; t < T; ++t) {
    const int64_t y = target[t];
    loss[t] = 0.0f;
    lse[t] = 0.0f;
    if (y == ignore) continue;
    if (y < 0 || y >= V) {
      *status = 1;
      continue;
    }
    const float* r = logits + t * V;
    double m = -INFINITY, d = 0.0;
    for (int64_t v = 0; v < V; ++v)
      if (r[v] > m) m = r[v];
    for (int64_t v = 0; v < V; ++v) d += exp((double)r[v] - m);
    lse[t] = (float)(m + log(d));
    loss[t] = (float)(m + log(d) - r[y]);
  }
}
