/*
 * Plain-C (float32, OpenMP) restatement of the fused sequence-mixing ops —
 * TEST INFRASTRUCTURE ONLY: the timed CPU baseline of bench.py and a second
 * checker for tests.  Never linked into the product library.
 *
 * Each function follows the same reference semantics as oracle/scans.py (which
 * cites the reference file:line for every formula) and is checked against it in
 * tests/test_oracle_cref.py.  Parallelism: OpenMP over independent
 * (batch, channel) or (batch, head) units, as a multi-core Nx/EXLA CPU run of the
 * reference's fallback tier would use.
 */
#include <math.h>
#include <stdlib.h>
#include <string.h>

#define DT_MIN 1.0e-3f
#define DT_MAX 0.1f

static float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }
static float sigm(float x) { return 1.0f / (1.0f + expf(-x)); }

/* The number of threads the parallel regions below actually run with (the team size of a
 * parallel region under the same settings). */
int cref_threads(void) {
#ifdef _OPENMP
  extern int omp_get_num_threads(void);
  int n = 1;
#pragma omp parallel
  {
#pragma omp single
    n = omp_get_num_threads();
  }
  return n;
#else
  return 1;
#endif
}

/* ---- MinGRU (post-sigmoid z, explicit h0; fused_scan.ex:516-528, 548-581) ---- */
void cref_mingru_fwd(const float* z, const float* c, const float* h0, float* out, int B, int T, int H) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      float s = h0 ? h0[(long)b * H + h] : 0.0f;
      for (int t = 0; t < T; ++t) {
        const long i = ((long)b * T + t) * H + h;
        s = (1.0f - z[i]) * s + z[i] * c[i];
        out[i] = s;
      }
    }
}

void cref_mingru_bwd(const float* z, const float* c, const float* h0, const float* fwd, const float* dy, float* dz,
                     float* dc, float* dh0, int B, int T, int H) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < H; ++h) {
      float carry = 0.0f;
      const float hz = h0 ? h0[(long)b * H + h] : 0.0f;
      for (int t = T - 1; t >= 0; --t) {
        const long i = ((long)b * T + t) * H + h;
        const float g = dy[i] + carry;
        const float hp = t > 0 ? fwd[i - H] : hz;
        dz[i] = g * (c[i] - hp);
        dc[i] = g * z[i];
        carry = g * (1.0f - z[i]);
      }
      if (dh0) dh0[(long)b * H + h] = carry;
    }
}

/* ---- selective scan, per-channel dt (fused_selective_scan.cu:41-91), with
 *      optional D skip and silu(z) gate ---- */
void cref_selective_scan_fwd(const float* x, const float* dt, const float* A, const float* Bm, const float* Cm,
                             const float* Dv, const float* z, float* out, int B, int T, int D, int N) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int b = 0; b < B; ++b)
    for (int d = 0; d < D; ++d) {
      float h[64];
      for (int n = 0; n < N; ++n) h[n] = 0.0f;
      for (int t = 0; t < T; ++t) {
        const long i = ((long)b * T + t) * D + d;
        const float dtc = clampf(dt[i], DT_MIN, DT_MAX);
        const float* Bt = Bm + ((long)b * T + t) * N;
        const float* Ct = Cm + ((long)b * T + t) * N;
        float y = 0.0f;
        for (int n = 0; n < N; ++n) {
          h[n] = expf(dtc * A[(long)d * N + n]) * h[n] + dtc * Bt[n] * x[i];
          y += Ct[n] * h[n];
        }
        if (Dv) y += Dv[d] * x[i];
        if (z) y *= z[i] * sigm(z[i]);
        out[i] = y;
      }
    }
}

/* backward (fused_scan.ex:1453-1533 plus dA, dD, dz).  dB, dC, dA, dD must be
 * zeroed by the caller; they are accumulated. */
void cref_selective_scan_bwd(const float* x, const float* dt, const float* A, const float* Bm, const float* Cm,
                             const float* Dv, const float* z, const float* dout, float* dx, float* ddt, float* dA,
                             float* dB, float* dC, float* dD, float* dz, int B, int T, int D, int N) {
  for (int b = 0; b < B; ++b) {
#pragma omp parallel
    {
      float* hs = (float*)malloc(sizeof(float) * (size_t)(T + 1) * N);
      float* lB = (float*)calloc((size_t)T * N, sizeof(float));
      float* lC = (float*)calloc((size_t)T * N, sizeof(float));
#pragma omp for schedule(static)
      for (int d = 0; d < D; ++d) {
        for (int n = 0; n < N; ++n) hs[n] = 0.0f;
        for (int t = 0; t < T; ++t) {  // recompute states: hs[(t+1)N + n] = h after step t
          const long i = ((long)b * T + t) * D + d;
          const float dtc = clampf(dt[i], DT_MIN, DT_MAX);
          const float* Bt = Bm + ((long)b * T + t) * N;
          for (int n = 0; n < N; ++n)
            hs[(long)(t + 1) * N + n] = expf(dtc * A[(long)d * N + n]) * hs[(long)t * N + n] + dtc * Bt[n] * x[i];
        }
        float dh[64], dAl[64];
        for (int n = 0; n < N; ++n) dh[n] = dAl[n] = 0.0f;
        float dDl = 0.0f;
        for (int t = T - 1; t >= 0; --t) {
          const long i = ((long)b * T + t) * D + d;
          const float dtr = dt[i];
          const float dtc = clampf(dtr, DT_MIN, DT_MAX);
          const float* Bt = Bm + ((long)b * T + t) * N;
          const float* Ct = Cm + ((long)b * T + t) * N;
          float g = dout[i];
          if (z) {
            float y = Dv ? Dv[d] * x[i] : 0.0f;
            for (int n = 0; n < N; ++n) y += Ct[n] * hs[(long)(t + 1) * N + n];
            const float sg = sigm(z[i]);
            dz[i] = g * y * sg * (1.0f + z[i] * (1.0f - sg));
            g = g * z[i] * sg;
          }
          float gx = Dv ? g * Dv[d] : 0.0f, gdt = 0.0f;
          dDl += g * x[i];
          for (int n = 0; n < N; ++n) {
            const float a = expf(dtc * A[(long)d * N + n]);
            const float hp = hs[(long)t * N + n];
            dh[n] += g * Ct[n];
            lC[(long)t * N + n] += g * hs[(long)(t + 1) * N + n];
            gx += dh[n] * dtc * Bt[n];
            const float ga = dh[n] * hp * a;
            gdt += ga * A[(long)d * N + n] + dh[n] * Bt[n] * x[i];
            dAl[n] += ga * dtc;
            lB[(long)t * N + n] += dh[n] * x[i] * dtc;
            dh[n] *= a;
          }
          dx[i] = gx;
          ddt[i] = (dtr >= DT_MIN && dtr <= DT_MAX) ? gdt : 0.0f;
        }
        for (int n = 0; n < N; ++n) dA[(long)d * N + n] += dAl[n];
        if (dD) dD[d] += dDl;
      }
#pragma omp critical
      {
        for (long j = 0; j < (long)T * N; ++j) {
          dB[(long)b * T * N + j] += lB[j];
          dC[(long)b * T * N + j] += lC[j];
        }
      }
      free(hs);
      free(lB);
      free(lC);
    }
  }
}
