/* Plain-C fp32 restatement of the scan recurrences -- TEST INFRASTRUCTURE.
 *
 * Used only as the timed CPU baseline ("port") of bench.py and cross-checked
 * against the float64 numpy oracle by the CPU tests.  Sequential over time,
 * OpenMP-parallel over independent rows, fp32 arithmetic with libm expf /
 * expm1f.  Never linked into or called by the product library.
 *
 * oc_multihead_scan  multihead_ssm_kernel.py:54-93,141-187 (DIAG family):
 *   per (b, head, p): Abar = exp(dt[b,t,h] a[h,p]), a = -exp(A_log);
 *   input term dt*B*u (Euler, :73-82) or expm1(dt a)/a * B * u (ZOH,
 *   discretize_kernel.py:50-54); y_head = sum_p C h + sum_p D u broadcast.
 * oc_ssd_scan        SSD: scalar a per head, state [P,N] per (b, head).
 * oc_selective_scan  Mamba-1 lanes (d, n), dt per (b, t).
 * oc_ssd_stream_step one streaming SSD step, state updated in place.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static inline float coef(int zoh, float dt, float a) {
  if (!zoh) return dt;
  float x = dt * a;
  return x == 0.0f ? dt : expm1f(x) / a;
}

int oc_num_threads(void) {
#ifdef _OPENMP
  extern int omp_get_max_threads(void);
  return omp_get_max_threads();
#else
  return 1;
#endif
}

/* u [Bsz,L,nh*hd]; A_log [nh*hd] (per channel) or [nh] (per_head);
 * B, C [Bsz,L,nh,hd]; dt [Bsz,L,nh]; D [nh*hd] or NULL; y [Bsz,L,nh*hd];
 * h_last [Bsz,nh,hd] or NULL.  All contiguous fp32. */
void oc_multihead_scan(int zoh, int per_head, const float* u, const float* A_log, const float* B,
                       const float* C, const float* dt, const float* D, float* y, float* h_last,
                       int64_t Bsz, int64_t L, int64_t nh, int64_t hd) {
  const int64_t H = nh * hd;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bsz; ++b) {
    for (int64_t h = 0; h < nh; ++h) {
      float* s = (float*)calloc((size_t)hd, sizeof(float));
      float* a = (float*)malloc((size_t)hd * sizeof(float));
      for (int64_t p = 0; p < hd; ++p) a[p] = -expf(A_log[per_head ? h : h * hd + p]);
      for (int64_t t = 0; t < L; ++t) {
        const float d = dt[(b * L + t) * nh + h];
        const float* ur = u + (b * L + t) * H + h * hd;
        const float* br = B + ((b * L + t) * nh + h) * hd;
        const float* cr = C + ((b * L + t) * nh + h) * hd;
        float acc = 0.0f;
        for (int64_t p = 0; p < hd; ++p) {
          const float ab = expf(d * a[p]);
          s[p] = ab * s[p] + coef(zoh, d, a[p]) * br[p] * ur[p];
          acc += cr[p] * s[p];
          if (D) acc += D[h * hd + p] * ur[p];
        }
        float* yr = y + (b * L + t) * H + h * hd;
        for (int64_t p = 0; p < hd; ++p) yr[p] = acc;
      }
      if (h_last) memcpy(h_last + (b * nh + h) * hd, s, (size_t)hd * sizeof(float));
      free(s);
      free(a);
    }
  }
}

/* x [Bsz,L,H,P]; dt [Bsz,L,H]; A_log [H]; B, C [Bsz,L,H,N]; D [H*P] or NULL;
 * h0 [Bsz,H,P,N] or NULL; y [Bsz,L,H,P]; h_last [Bsz,H,P,N] or NULL. */
void oc_ssd_scan(int zoh, const float* x, const float* dt, const float* A_log, const float* B,
                 const float* C, const float* D, const float* h0, float* y, float* h_last,
                 int64_t Bsz, int64_t L, int64_t H, int64_t P, int64_t N) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bsz; ++b) {
    for (int64_t h = 0; h < H; ++h) {
      float* s = (float*)malloc((size_t)(P * N) * sizeof(float));
      if (h0) memcpy(s, h0 + (b * H + h) * P * N, (size_t)(P * N) * sizeof(float));
      else memset(s, 0, (size_t)(P * N) * sizeof(float));
      const float a = -expf(A_log[h]);
      for (int64_t t = 0; t < L; ++t) {
        const float d = dt[(b * L + t) * H + h];
        const float ab = expf(d * a), cf = coef(zoh, d, a);
        const float* xr = x + ((b * L + t) * H + h) * P;
        const float* br = B + ((b * L + t) * H + h) * N;
        const float* cr = C + ((b * L + t) * H + h) * N;
        float* yr = y + ((b * L + t) * H + h) * P;
        for (int64_t p = 0; p < P; ++p) {
          float* sp = s + p * N;
          const float xv = cf * xr[p];
          float acc = D ? D[h * P + p] * xr[p] : 0.0f;
          for (int64_t n = 0; n < N; ++n) {
            sp[n] = ab * sp[n] + xv * br[n];
            acc += cr[n] * sp[n];
          }
          yr[p] = acc;
        }
      }
      if (h_last) memcpy(h_last + (b * H + h) * P * N, s, (size_t)(P * N) * sizeof(float));
      free(s);
    }
  }
}

/* x [Bsz,L,Dc]; dt [Bsz,L]; A_log [Dc,N]; B, C [Bsz,L,N]; D [Dc] or NULL;
 * y [Bsz,L,Dc]; h_last [Bsz,Dc,N] or NULL. */
void oc_selective_scan(int zoh, const float* x, const float* dt, const float* A_log,
                       const float* B, const float* C, const float* D, float* y, float* h_last,
                       int64_t Bsz, int64_t L, int64_t Dc, int64_t N) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bsz; ++b) {
    for (int64_t c = 0; c < Dc; ++c) {
      float* s = (float*)calloc((size_t)N, sizeof(float));
      float* a = (float*)malloc((size_t)N * sizeof(float));
      for (int64_t n = 0; n < N; ++n) a[n] = -expf(A_log[c * N + n]);
      for (int64_t t = 0; t < L; ++t) {
        const float d = dt[b * L + t];
        const float xv = x[(b * L + t) * Dc + c];
        const float* br = B + (b * L + t) * N;
        const float* cr = C + (b * L + t) * N;
        float acc = D ? D[c] * xv : 0.0f;
        for (int64_t n = 0; n < N; ++n) {
          s[n] = expf(d * a[n]) * s[n] + coef(zoh, d, a[n]) * br[n] * xv;
          acc += cr[n] * s[n];
        }
        y[(b * L + t) * Dc + c] = acc;
      }
      if (h_last) memcpy(h_last + (b * Dc + c) * N, s, (size_t)N * sizeof(float));
      free(s);
      free(a);
    }
  }
}

/* x [S,H,P]; dt [S]; A_log [H]; B, C [S,H,N]; D [H*P] or NULL;
 * state [S,H,P,N] in place; y [S,H,P]. */
void oc_ssd_stream_step(int zoh, const float* x, const float* dt, const float* A_log,
                        const float* B, const float* C, const float* D, float* state, float* y,
                        int64_t S, int64_t H, int64_t P, int64_t N) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t s = 0; s < S; ++s) {
    for (int64_t h = 0; h < H; ++h) {
      const float a = -expf(A_log[h]);
      const float d = dt[s];
      const float ab = expf(d * a), cf = coef(zoh, d, a);
      const float* br = B + (s * H + h) * N;
      const float* cr = C + (s * H + h) * N;
      for (int64_t p = 0; p < P; ++p) {
        float* sp = state + ((s * H + h) * P + p) * N;
        const float xv = x[(s * H + h) * P + p];
        float acc = D ? D[h * P + p] * xv : 0.0f;
        for (int64_t n = 0; n < N; ++n) {
          sp[n] = ab * sp[n] + cf * xv * br[n];
          acc += cr[n] * sp[n];
        }
        y[(s * H + h) * P + p] = acc;
      }
    }
  }
}

/* Time-aware interpolation, fused_interp_kernel.py:29-100 (fp32): for each
 * (b, t, FTILE-wide tile) the nearest step within K on each side whose tile
 * has any observed lane (mask tile sum > 0.5); time-weighted linear
 * interpolation, w = 0.5 when tau_next - tau_prev <= 1e-9.
 * V, M, Vhat [Bsz,T,F]; tau [Bsz,T]; contiguous fp32. */
void oc_time_aware_interp(const float* V, const float* M, const float* tau, float* Vhat,
                          int64_t Bsz, int64_t T, int64_t F, int64_t K, int64_t FTILE) {
  const int64_t nt = (F + FTILE - 1) / FTILE;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < Bsz; ++b) {
    for (int64_t tile = 0; tile < nt; ++tile) {
      const int64_t f0 = tile * FTILE, f1 = f0 + FTILE < F ? f0 + FTILE : F;
      unsigned char* obs = (unsigned char*)malloc((size_t)T);
      for (int64_t t = 0; t < T; ++t) {
        float s = 0.0f;
        for (int64_t f = f0; f < f1; ++f) s += M[(b * T + t) * F + f];
        obs[t] = s > 0.5f;
      }
      for (int64_t t = 0; t < T; ++t) {
        int64_t prev = -1, next = -1;
        for (int64_t k = 1; k <= K && prev < 0; ++k)
          if (t - k >= 0 && obs[t - k]) prev = t - k;
        for (int64_t k = 1; k <= K && next < 0; ++k)
          if (t + k < T && obs[t + k]) next = t + k;
        const float tp = prev >= 0 ? tau[b * T + prev] : 0.0f;
        const float tn = next >= 0 ? tau[b * T + next] : 0.0f;
        const float den = tn - tp;
        float w = den > 1e-9f ? (tau[b * T + t] - tp) / den : 0.5f;
        w = w < 0.0f ? 0.0f : (w > 1.0f ? 1.0f : w);
        const float* vr = V + b * T * F;
        float* o = Vhat + (b * T + t) * F;
        for (int64_t f = f0; f < f1; ++f) {
          float v;
          if (prev >= 0 && next >= 0) v = (1.0f - w) * vr[prev * F + f] + w * vr[next * F + f];
          else if (prev >= 0) v = vr[prev * F + f];
          else if (next >= 0) v = vr[next * F + f];
          else v = vr[t * F + f];
          o[f] = v;
        }
      }
      free(obs);
    }
  }
}
