/*
 * attention_oracle.c -- C statement of the attention forward math.
 * TEST INFRASTRUCTURE ONLY: loaded by tests/ (through oracle/c_oracle.py) as
 * a second, independent checker; never linked into the product.
 *
 * oracle_attention_ld: long-double two-pass softmax attention
 *   (softmax(scale*QK^T + mask) V), the closed form that the reference's
 *   fp32 path src/reference/attention_ref.py:10-45 approximates, plus the
 *   natural-log row LSE.  GQA: query head h reads KV head h/(Hq/Hkv)
 *   (reference src/flash_attention_sm75/ops.py:24-26).
 *
 * oracle_online_f32: fp32 tiled online softmax in the order of the
 *   reference scalar kernel src/kernels/flash_attention_forward.cu:48-163:
 *   running max initialised to -FLT_MAX, alpha = 0 while the max is
 *   -FLT_MAX (:131), masked keys skipped (:104-113,:139), o = o*alpha + p*v,
 *   final 1/l when l > 0 (:155).  With round_p != 0 each probability is
 *   rounded to fp16 before the PV product, as the WMMA kernels do (:495).
 *
 * Tensors are binary16 bit patterns, contiguous [B, H, N, D].
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* IEEE binary16 -> double, exact. */
static double h2d(uint16_t h) {
  const int sign = (h >> 15) & 1;
  const int exp = (h >> 10) & 0x1f;
  const int man = h & 0x3ff;
  double v;
  if (exp == 0) {
    v = ldexp((double)man, -24);
  } else if (exp == 31) {
    v = man ? NAN : INFINITY;
  } else {
    v = ldexp((double)(man | 0x400), exp - 25);
  }
  return sign ? -v : v;
}

/* float -> binary16 -> float with round-to-nearest-even (finite inputs). */
static float round_to_half(float f) {
  if (f == 0.0f || !isfinite(f)) return f;
  const float a = fabsf(f);
  if (a >= 65520.0f) return f > 0 ? INFINITY : -INFINITY;
  int e;
  frexpf(a, &e); /* a = m * 2^e, m in [0.5, 1) */
  /* spacing of binary16 values around a: 2^(e-11) for normals, 2^-24 below */
  int q = e - 11;
  if (q < -24) q = -24;
  const double step = ldexp(1.0, q);
  const double r = nearbyint((double)a / step) * step; /* default mode: RNE */
  return (float)(f < 0 ? -r : r);
}

void oracle_attention_ld(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         double* o, double* lse, int B, int Hq, int Hkv, int N,
                         int D, double scale, int causal) {
  const int group = Hq / Hkv;
  long double* s = (long double*)malloc(sizeof(long double) * (size_t)(N > 0 ? N : 1));
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const size_t qo = ((size_t)b * Hq + h) * (size_t)N * D;
      const size_t ko = ((size_t)b * Hkv + h / group) * (size_t)N * D;
      for (int i = 0; i < N; ++i) {
        const int last = causal ? i : N - 1;
        long double m = -INFINITY;
        for (int j = 0; j <= last; ++j) {
          long double acc = 0.0L;
          for (int d = 0; d < D; ++d)
            acc += (long double)h2d(q[qo + (size_t)i * D + d]) *
                   (long double)h2d(k[ko + (size_t)j * D + d]);
          s[j] = acc * (long double)scale;
          if (s[j] > m) m = s[j];
        }
        long double l = 0.0L;
        for (int j = 0; j <= last; ++j) {
          s[j] = expl(s[j] - m);
          l += s[j];
        }
        for (int d = 0; d < D; ++d) {
          long double acc = 0.0L;
          for (int j = 0; j <= last; ++j)
            acc += s[j] * (long double)h2d(v[ko + (size_t)j * D + d]);
          o[qo + (size_t)i * D + d] = (double)(acc / l);
        }
        if (lse) lse[((size_t)b * Hq + h) * N + i] = (double)(m + logl(l));
      }
    }
  free(s);
}

void oracle_online_f32(const uint16_t* q, const uint16_t* k, const uint16_t* v,
                       float* o, int B, int Hq, int Hkv, int N, int D, float scale,
                       int causal, int tile, int round_p) {
  const int group = Hq / Hkv;
  float* acc = (float*)malloc(sizeof(float) * (size_t)D);
  float* sc = (float*)malloc(sizeof(float) * (size_t)tile);
  for (int b = 0; b < B; ++b)
    for (int h = 0; h < Hq; ++h) {
      const size_t qo = ((size_t)b * Hq + h) * (size_t)N * D;
      const size_t ko = ((size_t)b * Hkv + h / group) * (size_t)N * D;
      for (int i = 0; i < N; ++i) {
        float mi = -FLT_MAX, li = 0.0f;
        for (int d = 0; d < D; ++d) acc[d] = 0.0f;
        for (int k0 = 0; k0 < N; k0 += tile) {
          if (causal && k0 > i) break;
          float mij = -FLT_MAX;
          for (int c = 0; c < tile; ++c) {
            const int j = k0 + c;
            if (j >= N || (causal && j > i)) {
              sc[c] = -FLT_MAX;
              continue;
            }
            float s = 0.0f;
            for (int d = 0; d < D; ++d)
              s += (float)h2d(q[qo + (size_t)i * D + d]) * (float)h2d(k[ko + (size_t)j * D + d]);
            sc[c] = s * scale;
            if (sc[c] > mij) mij = sc[c];
          }
          const float mn = mi > mij ? mi : mij;
          const float alpha = (mi == -FLT_MAX) ? 0.0f : expf(mi - mn);
          for (int d = 0; d < D; ++d) acc[d] *= alpha;
          float lij = 0.0f;
          for (int c = 0; c < tile; ++c) {
            if (sc[c] == -FLT_MAX) continue;
            float p = expf(sc[c] - mn);
            lij += p;
            if (round_p) p = round_to_half(p);
            const int j = k0 + c;
            for (int d = 0; d < D; ++d) acc[d] += p * (float)h2d(v[ko + (size_t)j * D + d]);
          }
          li = li * alpha + lij;
          mi = mn;
        }
        const float inv = li > 0.0f ? 1.0f / li : 0.0f;
        for (int d = 0; d < D; ++d) o[qo + (size_t)i * D + d] = acc[d] * inv;
      }
    }
  free(sc);
  free(acc);
}

/* glibc rand() streams used by the reference's own harnesses, exposed so the
 * fixture generator reproduces their inputs bit-for-bit. */
void oracle_rand_stream(unsigned seed, int n, float lo_scale, float* out) {
  /* value = (rand()/RAND_MAX - 0.5) * lo_scale */
  srand(seed);
  for (int i = 0; i < n; ++i) out[i] = ((float)rand() / (float)RAND_MAX - 0.5f) * lo_scale;
}

/* One row-block softmax of a 16x16 tile as in reference
 * fused/src/test_warp_softmax.cu (scale, row max, exp, row sum; optionally
 * normalised), double precision. */
void oracle_tile_softmax(const float* in, double* out, double* row_max, double* row_sum,
                         int rows, int cols, double scale, int normalize) {
  for (int r = 0; r < rows; ++r) {
    double m = -INFINITY;
    for (int c = 0; c < cols; ++c) {
      const double x = (double)in[r * cols + c] * scale;
      if (x > m) m = x;
    }
    double s = 0.0;
    for (int c = 0; c < cols; ++c) {
      out[r * cols + c] = exp((double)in[r * cols + c] * scale - m);
      s += out[r * cols + c];
    }
    if (normalize)
      for (int c = 0; c < cols; ++c) out[r * cols + c] /= s;
    row_max[r] = m;
    row_sum[r] = s;
  }
}
