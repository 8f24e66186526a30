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

/* ---- delta rule, recurrent form (delta_net.ex:231-273; gated_delta_net.ex:300-353) ----
 * q, k, v, out: [B, T, H, d] (d_k = d_v = d); beta: [B, T, H] (per head) when beta_per_head,
 * else [B, T, H, d] (per value row); alpha: [B, T, H] or NULL (DeltaNet).  State S[d_v][d_k]
 * per (b, h): S = a S; e = beta (v - S k); S += e k^T; o = S q, fused row by row. */
static float dr_beta(const float* beta, int per_head, long bth, int i, int d) {
  return per_head ? beta[bth] : beta[bth * d + i];
}

static void dr_head_fwd(const float* q, const float* k, const float* v, const float* beta, const float* alpha,
                        float* out, float* S, float* ckpt, int ck, int b, int h, int T, int H, int d,
                        int beta_per_head) {
  memset(S, 0, sizeof(float) * (size_t)d * d);
  for (int t = 0; t < T; ++t) {
    if (ckpt && t % ck == 0) memcpy(ckpt + (size_t)(t / ck) * d * d, S, sizeof(float) * (size_t)d * d);
    const long bth = ((long)b * T + t) * H + h;
    const float* kt = k + bth * d;
    const float* qt = q + bth * d;
    const float* vt = v + bth * d;
    const float a = alpha ? alpha[bth] : 1.0f;
    for (int i = 0; i < d; ++i) {
      float* Si = S + (size_t)i * d;
      float r = 0.0f;
#pragma omp simd reduction(+ : r)
      for (int j = 0; j < d; ++j) r += Si[j] * kt[j];
      const float e = dr_beta(beta, beta_per_head, bth, i, d) * (vt[i] - a * r);
      float o = 0.0f;
#pragma omp simd reduction(+ : o)
      for (int j = 0; j < d; ++j) {
        Si[j] = a * Si[j] + e * kt[j];
        o += Si[j] * qt[j];
      }
      if (out) out[bth * d + i] = o;
    }
  }
}

void cref_delta_rule_fwd(const float* q, const float* k, const float* v, const float* beta, const float* alpha,
                         float* out, int B, int T, int H, int d, int beta_per_head) {
#pragma omp parallel
  {
    float* S = (float*)malloc(sizeof(float) * (size_t)d * d);
#pragma omp for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h) dr_head_fwd(q, k, v, beta, alpha, out, S, NULL, 1, b, h, T, H, d, beta_per_head);
    free(S);
  }
}

/* Reverse pass (fused_scan.ex:1257-1328, 1347-1431), with the states every CK steps saved by
 * a forward pass and each chunk's states recomputed from its checkpoint.  dbeta has beta's
 * layout; dalpha [B, T, H] (ignored when alpha is NULL). */
#define DR_CK 64
void cref_delta_rule_bwd(const float* q, const float* k, const float* v, const float* beta, const float* alpha,
                         const float* dout, float* dq, float* dk, float* dv, float* dbeta, float* dalpha, int B,
                         int T, int H, int d, int beta_per_head) {
  const int nck = (T + DR_CK - 1) / DR_CK;
  const size_t dd = (size_t)d * d;
#pragma omp parallel
  {
    float* S = (float*)malloc(sizeof(float) * dd);
    float* ck = (float*)malloc(sizeof(float) * dd * nck);
    float* st = (float*)malloc(sizeof(float) * dd * DR_CK);  /* S_{t-1} of each step of a chunk */
    float* dS = (float*)malloc(sizeof(float) * dd);
    float* err = (float*)malloc(sizeof(float) * d);
    float* dsk = (float*)malloc(sizeof(float) * d);
    float* dkt = (float*)malloc(sizeof(float) * d);
    float* dqt = (float*)malloc(sizeof(float) * d);
#pragma omp for collapse(2) schedule(static)
    for (int b = 0; b < B; ++b)
      for (int h = 0; h < H; ++h) {
        dr_head_fwd(q, k, v, beta, alpha, NULL, S, ck, DR_CK, b, h, T, H, d, beta_per_head);
        memset(dS, 0, sizeof(float) * dd);
        for (int c = nck - 1; c >= 0; --c) {
          const int t0 = c * DR_CK, t1 = t0 + DR_CK < T ? t0 + DR_CK : T;
          memcpy(S, ck + (size_t)c * dd, sizeof(float) * dd);
          for (int t = t0; t < t1; ++t) {  /* states entering each step of the chunk */
            memcpy(st + (size_t)(t - t0) * dd, S, sizeof(float) * dd);
            const long bth = ((long)b * T + t) * H + h;
            const float* kt = k + bth * d;
            const float a = alpha ? alpha[bth] : 1.0f;
            for (int i = 0; i < d; ++i) {
              float* Si = S + (size_t)i * d;
              float r = 0.0f;
#pragma omp simd reduction(+ : r)
              for (int j = 0; j < d; ++j) r += Si[j] * kt[j];
              const float e = dr_beta(beta, beta_per_head, bth, i, d) * (v[bth * d + i] - a * r);
#pragma omp simd
              for (int j = 0; j < d; ++j) Si[j] = a * Si[j] + e * kt[j];
            }
          }
          for (int t = t1 - 1; t >= t0; --t) {
            const float* sp = st + (size_t)(t - t0) * dd;
            const long bth = ((long)b * T + t) * H + h;
            const float *kt = k + bth * d, *qt = q + bth * d, *vt = v + bth * d, *dot = dout + bth * d;
            const float a = alpha ? alpha[bth] : 1.0f;
            for (int i = 0; i < d; ++i) {  /* err = v - (a S_{t-1}) k */
              float r = 0.0f;
#pragma omp simd reduction(+ : r)
              for (int j = 0; j < d; ++j) r += sp[(size_t)i * d + j] * kt[j];
              err[i] = vt[i] - a * r;
            }
            for (int j = 0; j < d; ++j) dqt[j] = dkt[j] = 0.0f;
            float dbh = 0.0f, dal = 0.0f;
            for (int i = 0; i < d; ++i) {  /* dq = S_t^T do; ds_k = dtot k; dk += dtot^T (beta err) */
              const float bi = dr_beta(beta, beta_per_head, bth, i, d);
              const float be = bi * err[i], doi = dot[i];
              const float* spi = sp + (size_t)i * d;
              const float* dSi = dS + (size_t)i * d;
              float s = 0.0f;
#pragma omp simd reduction(+ : s)
              for (int j = 0; j < d; ++j) {
                dqt[j] += (a * spi[j] + be * kt[j]) * doi;
                const float dtot = dSi[j] + doi * qt[j];
                s += dtot * kt[j];
                dkt[j] += dtot * be;
              }
              dsk[i] = s;
              dv[bth * d + i] = bi * s;
              if (beta_per_head) dbh += err[i] * s;
              else dbeta[bth * d + i] = err[i] * s;
            }
            for (int i = 0; i < d; ++i) {  /* d_dec = dtot - beta ds_k k^T; dk -= (a S_{t-1})^T beta ds_k */
              const float bs = dr_beta(beta, beta_per_head, bth, i, d) * dsk[i], doi = dot[i];
              const float* spi = sp + (size_t)i * d;
              float* dSi = dS + (size_t)i * d;
              float acc = 0.0f;
#pragma omp simd reduction(+ : acc)
              for (int j = 0; j < d; ++j) {
                const float ddec = dSi[j] + doi * qt[j] - bs * kt[j];
                acc += ddec * spi[j];
                dkt[j] -= a * spi[j] * bs;
                dSi[j] = a * ddec;
              }
              dal += acc;
            }
            for (int j = 0; j < d; ++j) {
              dq[bth * d + j] = dqt[j];
              dk[bth * d + j] = dkt[j];
            }
            if (beta_per_head) dbeta[bth] = dbh;
            if (alpha && dalpha) dalpha[bth] = dal;
          }
        }
      }
    free(S); free(ck); free(st); free(dS); free(err); free(dsk); free(dkt); free(dqt);
  }
}

/* ---- softmax attention (fused_scan.ex:3476-3508, backward 3527-3570) ----
 * q, k, v, out, dout, dq, dk, dv: [BH, T, d]; lse [BH, T] (natural log of the scaled scores);
 * scale 1 / sqrt(d); causal keeps key j <= query i. */
void cref_attention_fwd(const float* q, const float* k, const float* v, float* out, float* lse, int BH, int T, int d,
                        int causal) {
  const float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel
  {
    float* p = (float*)malloc(sizeof(float) * T);
    float* o = (float*)malloc(sizeof(float) * d);
#pragma omp for collapse(2) schedule(dynamic, 16)
    for (int bh = 0; bh < BH; ++bh)
      for (int i = 0; i < T; ++i) {
        const float* qi = q + ((long)bh * T + i) * d;
        const int nk = causal ? i + 1 : T;
        float m = -INFINITY;
        for (int j = 0; j < nk; ++j) {
          const float* kj = k + ((long)bh * T + j) * d;
          float s = 0.0f;
#pragma omp simd reduction(+ : s)
          for (int e = 0; e < d; ++e) s += qi[e] * kj[e];
          p[j] = s * scale;
          m = p[j] > m ? p[j] : m;
        }
        float l = 0.0f;
        for (int e = 0; e < d; ++e) o[e] = 0.0f;
        for (int j = 0; j < nk; ++j) {
          const float w = expf(p[j] - m);
          l += w;
          const float* vj = v + ((long)bh * T + j) * d;
#pragma omp simd
          for (int e = 0; e < d; ++e) o[e] += w * vj[e];
        }
        float* oi = out + ((long)bh * T + i) * d;
        for (int e = 0; e < d; ++e) oi[e] = o[e] / l;
        lse[(long)bh * T + i] = m + logf(l);
      }
    free(p);
    free(o);
  }
}

void cref_attention_bwd(const float* q, const float* k, const float* v, const float* out, const float* dout,
                        const float* lse, float* dq, float* dk, float* dv, int BH, int T, int d, int causal) {
  const float scale = 1.0f / sqrtf((float)d);
#pragma omp parallel for schedule(dynamic, 1)
  for (int bh = 0; bh < BH; ++bh) {
    const long base = (long)bh * T * d;
    memset(dk + base, 0, sizeof(float) * (size_t)T * d);
    memset(dv + base, 0, sizeof(float) * (size_t)T * d);
    for (int i = 0; i < T; ++i) {
      const float *qi = q + base + (long)i * d, *doi = dout + base + (long)i * d, *oi = out + base + (long)i * d;
      float Di = 0.0f;
      for (int e = 0; e < d; ++e) Di += doi[e] * oi[e];
      float* dqi = dq + base + (long)i * d;
      for (int e = 0; e < d; ++e) dqi[e] = 0.0f;
      const int nk = causal ? i + 1 : T;
      const float li = lse[(long)bh * T + i];
      for (int j = 0; j < nk; ++j) {
        const float *kj = k + base + (long)j * d, *vj = v + base + (long)j * d;
        float s = 0.0f, dp = 0.0f;
#pragma omp simd reduction(+ : s, dp)
        for (int e = 0; e < d; ++e) {
          s += qi[e] * kj[e];
          dp += doi[e] * vj[e];
        }
        const float pij = expf(s * scale - li);
        const float ds = pij * (dp - Di) * scale;
        float *dkj = dk + base + (long)j * d, *dvj = dv + base + (long)j * d;
#pragma omp simd
        for (int e = 0; e < d; ++e) {
          dqi[e] += ds * kj[e];
          dkj[e] += ds * qi[e];
          dvj[e] += pij * doi[e];
        }
      }
    }
  }
}
