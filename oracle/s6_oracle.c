/*
 * CPU restatement of the S6 selective scan in C -- TEST INFRASTRUCTURE ONLY.
 *
 * Used by tests/ (full-size parity checks) and by bench.py's cpu_baseline leg; never by
 * the product library.  It follows the reference CPU path selective_scan_ref
 * (/root/reference/zoology/zoology/mixers/mamba_ssm/ops/selective_scan_interface.py:107-156)
 * with the same fp32 rounding points, one channel (b, d) at a time instead of
 * materialising the [B, D, L, N] tensors:
 *   delta += bias; delta = softplus(delta)            (109-112, threshold 20)
 *   deltaA   = expf(delta * A)                        (126)
 *   deltaB_u = (delta * B) * u                        (131; einsum contracts left to right)
 *   x = deltaA * x + deltaB_u   (separate multiply and add, no FMA contraction)   (139)
 *   y = sum_n x * C   (accumulated in n order)         (144)
 *   out = y + u * D;  out *= silu(z)                   (153-155)
 * The caller casts `out` to the input dtype (156).
 *
 * The backward is the hand-derived reverse recurrence of oracle/brute64.py evaluated in
 * double precision from the fp32 inputs; tests/test_oracle.py checks it against autograd
 * through the torch restatement.  Varlen (cu_seqlens) resets the state at every sequence
 * start.  All arrays are dense row-major: u, delta, z, dout, out: [B, D, L];
 * A: [D, N]; Bm, Cm: [B, G, N, L]; D, bias: [D].
 *
 * Build: make -C oracle   (gcc -O2 -fopenmp -ffp-contract=off)
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static float softplus20f(float x) { return x <= 20.f ? log1pf(expf(x)) : x; }

static void starts_mask(int64_t L, const int32_t* cu, int32_t nseq, unsigned char* st) {
  memset(st, 0, (size_t)L);
  st[0] = 1;
  for (int32_t i = 0; i < nseq; ++i)
    if (cu[i] < L) st[cu[i]] = 1;
}

/* last_state: [B, D, N] (dense) or [nseq, D, N] (varlen); may be NULL. */
void s6o_fwd(int64_t Bsz, int64_t D, int64_t L, int64_t N, int64_t G, const float* u,
             const float* delta, const float* A, const float* Bm, const float* Cm,
             const float* Dv, const float* z, const float* bias, int softplus,
             const int32_t* cu, int32_t nseq, float* out, float* last_state) {
  unsigned char* st = (unsigned char*)malloc((size_t)L);
  starts_mask(L, cu, nseq > 0 ? nseq : 0, st);
  const int64_t Dg = D / G;
  if (last_state && nseq > 0)  /* empty sequences keep a zero final state */
    memset(last_state, 0, (size_t)(nseq * D * N) * sizeof(float));
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t ch = 0; ch < Bsz * D; ++ch) {
    const int64_t b = ch / D, d = ch % D, g = d / Dg;
    float* x = (float*)calloc((size_t)N, sizeof(float));
    const float* uu = u + ch * L;
    const float* dl = delta + ch * L;
    const float* Bb = Bm + (b * G + g) * N * L;
    const float* Cb = Cm + (b * G + g) * N * L;
    float* o = out + ch * L;
    const float bi = bias ? bias[d] : 0.f;
    int32_t seq = -1;
    for (int64_t t = 0; t < L; ++t) {
      if (st[t]) {
        memset(x, 0, (size_t)N * sizeof(float));
        ++seq;
        if (nseq > 0)
          while (seq + 1 < nseq && cu[seq + 1] <= t) ++seq;
      }
      float dt = dl[t];
      if (bias) dt = dt + bi;
      if (softplus) dt = softplus20f(dt);
      float y = 0.f;
      for (int64_t n = 0; n < N; ++n) {
        const float dA = expf(dt * A[d * N + n]);
        const float dBu = (dt * Bb[n * L + t]) * uu[t];
        const float prod = dA * x[n];
        x[n] = prod + dBu;
        const float c = x[n] * Cb[n * L + t];
        y = y + c;
      }
      float r = y;
      if (Dv) r = y + uu[t] * Dv[d];
      if (z) {
        const float zz = z[ch * L + t];
        r = r * (zz / (1.f + expf(-zz)));
      }
      o[t] = r;
      const int end = (t == L - 1) || (nseq > 0 && st[t + 1]);
      if (last_state && end) {
        const int64_t row = nseq > 0 ? ((int64_t)seq * D + d) : ch;
        for (int64_t n = 0; n < N; ++n) last_state[row * N + n] = x[n];
      }
    }
    free(x);
  }
  free(st);
}

static double sigm(double x) { return 1.0 / (1.0 + exp(-x)); }

/* Gradients of sum(out * dout).  dB, dC: [B, G, N, L]; dA: [D, N]; dD, dbias: [D] (may be
 * NULL when the input is absent); dz: [B, D, L] (NULL without z). */
void s6o_bwd(int64_t Bsz, int64_t D, int64_t L, int64_t N, int64_t G, const float* u,
             const float* delta, const float* A, const float* Bm, const float* Cm,
             const float* Dv, const float* z, const float* bias, int softplus,
             const int32_t* cu, int32_t nseq, const float* dout, float* du, float* ddelta,
             float* dA, float* dB, float* dC, float* dD, float* dz, float* dbias) {
  unsigned char* st = (unsigned char*)malloc((size_t)L);
  starts_mask(L, cu, nseq > 0 ? nseq : 0, st);
  const int64_t Dg = D / G;
  const size_t nbc = (size_t)(Bsz * G * N * L);
  double* accB = (double*)calloc(nbc, sizeof(double));
  double* accC = (double*)calloc(nbc, sizeof(double));
#pragma omp parallel
  {
    double* pB = (double*)calloc(nbc, sizeof(double));
    double* pC = (double*)calloc(nbc, sizeof(double));
    double* h = (double*)malloc((size_t)(L * N) * sizeof(double));
    double* Delta = (double*)malloc((size_t)L * sizeof(double));
    double* pre = (double*)malloc((size_t)L * sizeof(double));
    double* lam_next = (double*)malloc((size_t)N * sizeof(double));
    double* dAl = (double*)malloc((size_t)N * sizeof(double));
#pragma omp for schedule(dynamic, 1)
    for (int64_t d = 0; d < D; ++d) {
      const int64_t g = d / Dg;
      for (int64_t n = 0; n < N; ++n) dAl[n] = 0.0;
      double dDl = 0.0, dbl = 0.0;
      for (int64_t b = 0; b < Bsz; ++b) {
        const int64_t ch = b * D + d;
        const float* uu = u + ch * L;
        const float* Bb = Bm + (b * G + g) * N * L;
        const float* Cb = Cm + (b * G + g) * N * L;
        for (int64_t t = 0; t < L; ++t) {
          double p = (double)delta[ch * L + t] + (bias ? (double)bias[d] : 0.0);
          pre[t] = p;
          Delta[t] = softplus ? (p <= 20.0 ? log1p(exp(p)) : p) : p;
          for (int64_t n = 0; n < N; ++n) {
            const double hp = (st[t] || t == 0) ? 0.0 : h[(t - 1) * N + n];
            h[t * N + n] = exp(Delta[t] * A[d * N + n]) * hp + Delta[t] * uu[t] * Bb[n * L + t];
          }
        }
        for (int64_t n = 0; n < N; ++n) lam_next[n] = 0.0;
        for (int64_t t = L - 1; t >= 0; --t) {
          double dy = dout[ch * L + t];
          double y = 0.0;
          if (z) {
            for (int64_t n = 0; n < N; ++n) y += h[t * N + n] * Cb[n * L + t];
            if (Dv) y += (double)uu[t] * Dv[d];
            const double zz = z[ch * L + t], sg = sigm(zz);
            dz[ch * L + t] = (float)(dy * y * sg * (1.0 + zz * (1.0 - sg)));
            dy = dy * zz * sg;
          }
          double s1 = 0.0, s2 = 0.0;
          for (int64_t n = 0; n < N; ++n) {
            const double a = exp(Delta[t] * A[d * N + n]);
            const double lam = Cb[n * L + t] * dy + lam_next[n];
            const double hp = (st[t] || t == 0) ? 0.0 : h[(t - 1) * N + n];
            const double q = lam * a * hp;
            dAl[n] += q * Delta[t];
            s2 += q * A[d * N + n];
            s1 += lam * Bb[n * L + t];
            pB[((b * G + g) * N + n) * L + t] += lam * Delta[t] * uu[t];
            pC[((b * G + g) * N + n) * L + t] += h[t * N + n] * dy;
            lam_next[n] = st[t] ? 0.0 : a * lam;
          }
          double duv = s1 * Delta[t];
          if (Dv) {
            duv += dy * Dv[d];
            dDl += dy * uu[t];
          }
          double dd = s2 + s1 * uu[t];
          if (softplus) dd *= (pre[t] <= 20.0 ? sigm(pre[t]) : 1.0);
          du[ch * L + t] = (float)duv;
          ddelta[ch * L + t] = (float)dd;
          dbl += dd;
        }
      }
      for (int64_t n = 0; n < N; ++n) dA[d * N + n] = (float)dAl[n];
      if (dD) dD[d] = (float)dDl;
      if (dbias) dbias[d] = (float)dbl;
    }
#pragma omp critical
    {
      for (size_t i = 0; i < nbc; ++i) {
        accB[i] += pB[i];
        accC[i] += pC[i];
      }
    }
    free(pB); free(pC); free(h); free(Delta); free(pre); free(lam_next); free(dAl);
  }
  for (size_t i = 0; i < nbc; ++i) {
    dB[i] = (float)accB[i];
    dC[i] = (float)accC[i];
  }
  free(accB); free(accC); free(st);
}

/* The same recurrence evaluated in double precision from the fp32 inputs (no rounding to
 * fp32 anywhere): the exact value that the fp32 paths are compared with.  Same arguments as
 * s6o_fwd; out / last_state are double.  Pinned against oracle/brute64.py scan_fwd64. */
void s6o_fwd64(int64_t Bsz, int64_t D, int64_t L, int64_t N, int64_t G, const float* u,
               const float* delta, const float* A, const float* Bm, const float* Cm,
               const float* Dv, const float* z, const float* bias, int softplus,
               const int32_t* cu, int32_t nseq, double* out, double* last_state) {
  unsigned char* st = (unsigned char*)malloc((size_t)L);
  starts_mask(L, cu, nseq > 0 ? nseq : 0, st);
  const int64_t Dg = D / G;
  if (last_state && nseq > 0)
    memset(last_state, 0, (size_t)(nseq * D * N) * sizeof(double));
#pragma omp parallel for schedule(dynamic, 1)
  for (int64_t ch = 0; ch < Bsz * D; ++ch) {
    const int64_t b = ch / D, d = ch % D, g = d / Dg;
    double* x = (double*)calloc((size_t)N, sizeof(double));
    const float* uu = u + ch * L;
    const float* Bb = Bm + (b * G + g) * N * L;
    const float* Cb = Cm + (b * G + g) * N * L;
    int32_t seq = -1;
    for (int64_t t = 0; t < L; ++t) {
      if (st[t]) {
        memset(x, 0, (size_t)N * sizeof(double));
        ++seq;
        if (nseq > 0)
          while (seq + 1 < nseq && cu[seq + 1] <= t) ++seq;
      }
      double dt = (double)delta[ch * L + t] + (bias ? (double)bias[d] : 0.0);
      if (softplus) dt = dt <= 20.0 ? log1p(exp(dt)) : dt;
      double y = 0.0;
      for (int64_t n = 0; n < N; ++n) {
        x[n] = exp(dt * A[d * N + n]) * x[n] + dt * uu[t] * Bb[n * L + t];
        y += x[n] * Cb[n * L + t];
      }
      if (Dv) y += (double)uu[t] * Dv[d];
      if (z) {
        const double zz = z[ch * L + t];
        y *= zz / (1.0 + exp(-zz));
      }
      out[ch * L + t] = y;
      const int end = (t == L - 1) || (nseq > 0 && st[t + 1]);
      if (last_state && end) {
        const int64_t row = nseq > 0 ? ((int64_t)seq * D + d) : ch;
        for (int64_t n = 0; n < N; ++n) last_state[row * N + n] = x[n];
      }
    }
    free(x);
  }
  free(st);
}
