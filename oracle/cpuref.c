/*
 * C/OpenMP restatement of moelan's numba kernels for the routed-expert path.
 *
 * TEST INFRASTRUCTURE: the CPU baseline of bench.py (timed beside the GPU) and
 * an extra cross-check in tests/. The product library never links or calls it.
 *
 * Each function follows the loop structure of one numba kernel of moelan 0.1.0
 * (moelan/kernels.py), with `#pragma omp parallel for` where numba has prange
 * and -ffast-math where numba has fastmath=True, so the timing reflects the
 * reference's own CPU path on the same cores.
 */
#include <math.h>
#include <omp.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* _q4, moelan/kernels.py:85-106, and its wrapper q4_matmul_t :1018-1027:
 * unsigned nibbles against the even / odd input columns, then
 * y -= 8 * (group sums of x) @ s.T */
void ref_q4_matmul_t(const float* x, int n, const uint8_t* raw, const float* s, int O, int I, int gs, int xor8,
                     float* y) {
  const int half = gs / 2, ng = I / gs, C = I / 2;
  float* xe = (float*)malloc(sizeof(float) * (size_t)n * C);
  float* xo = (float*)malloc(sizeof(float) * (size_t)n * C);
  float* xsum = (float*)malloc(sizeof(float) * (size_t)n * ng);
  for (int r = 0; r < n; ++r) {
    for (int j = 0; j < C; ++j) {
      xe[(size_t)r * C + j] = x[(size_t)r * I + 2 * j];
      xo[(size_t)r * C + j] = x[(size_t)r * I + 2 * j + 1];
    }
    for (int g = 0; g < ng; ++g) {
      float a = 0.f;
      for (int j = 0; j < gs; ++j) a += x[(size_t)r * I + g * gs + j];
      xsum[(size_t)r * ng + g] = a;
    }
  }
#pragma omp parallel for schedule(static)
  for (int o = 0; o < O; ++o) {
    const uint8_t* row = raw + (size_t)o * C;
    for (int r = 0; r < n; ++r) {
      const float* e = xe + (size_t)r * C;
      const float* d = xo + (size_t)r * C;
      float acc = 0.f, corr = 0.f;
      for (int g = 0; g < ng; ++g) {
        float part = 0.f;
        const int b0 = g * half;
        for (int k = 0; k < half; ++k) {
          const int b = row[b0 + k] ^ xor8;
          part += (float)(b & 15) * e[b0 + k] + (float)(b >> 4) * d[b0 + k];
        }
        acc += part * s[(size_t)o * ng + g];
        corr += s[(size_t)o * ng + g] * xsum[(size_t)r * ng + g];
      }
      y[(size_t)r * O + o] = acc - 8.0f * corr;
    }
  }
  free(xe);
  free(xo);
  free(xsum);
}

/* _q8, moelan/kernels.py:152-168 */
void ref_q8_matmul_t(const float* x, int n, const int8_t* q, const float* s, int O, int I, int gs, float* y) {
  const int ng = I / gs;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < O; ++o) {
    for (int r = 0; r < n; ++r) {
      float acc = 0.f;
      for (int g = 0; g < ng; ++g) {
        float part = 0.f;
        const int x0 = g * gs;
        for (int k = 0; k < gs; ++k) part += (float)q[(size_t)o * I + x0 + k] * x[(size_t)r * I + x0 + k];
        acc += part * s[(size_t)o * ng + g];
      }
      y[(size_t)r * O + o] = acc;
    }
  }
}

/* _moe_q4, moelan/kernels.py:712-782: one layer's int4 experts for a few rows.
 * ptrs[4e..4e+3] = addresses of gate|up bytes, their f32 scales, down bytes,
 * their scales; pairs poff[e]..poff[e+1] with input row prow[p] (into xs) and
 * gate weight pw[p]; out [n_rows, H] is added to (part in the reference). */
void ref_moe_q4(const float* xs, int n_rows, const uint64_t* ptrs, const uint8_t* xors, const int64_t* poff,
                const int64_t* prow, const float* pw, int k, int P, int H, int I, int gs, float* out) {
  const int O1 = 2 * I, C1 = H / 2, G1 = H / gs, C2 = I / 2, G2 = I / gs, half = gs / 2;
  float* xe = (float*)malloc(sizeof(float) * (size_t)n_rows * C1);
  float* xo = (float*)malloc(sizeof(float) * (size_t)n_rows * C1);
  float* xsum = (float*)malloc(sizeof(float) * (size_t)n_rows * G1);
  for (int r = 0; r < n_rows; ++r) {
    for (int j = 0; j < C1; ++j) {
      xe[(size_t)r * C1 + j] = xs[(size_t)r * H + 2 * j];
      xo[(size_t)r * C1 + j] = xs[(size_t)r * H + 2 * j + 1];
    }
    for (int g = 0; g < G1; ++g) {
      float a = 0.f;
      for (int j = 0; j < gs; ++j) a += xs[(size_t)r * H + g * gs + j];
      xsum[(size_t)r * G1 + g] = a;
    }
  }
  float* h = (float*)malloc(sizeof(float) * (size_t)P * O1);
#pragma omp parallel for schedule(static)
  for (long t = 0; t < (long)k * O1; ++t) {
    const int e = (int)(t / O1), o = (int)(t - (long)e * O1);
    const uint8_t* raw = (const uint8_t*)(uintptr_t)ptrs[4 * e] + (size_t)o * C1;
    const float* sc = (const float*)(uintptr_t)ptrs[4 * e + 1] + (size_t)o * G1;
    const int xr = xors[e];
    for (int64_t p = poff[e]; p < poff[e + 1]; ++p) {
      const int64_t r = prow[p];
      float acc = 0.f, corr = 0.f;
      for (int g = 0; g < G1; ++g) {
        float part = 0.f;
        const int b0 = g * half;
        for (int j = 0; j < half; ++j) {
          const int b = raw[b0 + j] ^ xr;
          part += (float)(b & 15) * xe[r * C1 + b0 + j] + (float)(b >> 4) * xo[r * C1 + b0 + j];
        }
        acc += part * sc[g];
        corr += sc[g] * xsum[r * G1 + g];
      }
      h[(size_t)p * O1 + o] = acc - 8.0f * corr;
    }
  }
  float* ae = (float*)malloc(sizeof(float) * (size_t)P * C2);
  float* ao = (float*)malloc(sizeof(float) * (size_t)P * C2);
  float* asum = (float*)malloc(sizeof(float) * (size_t)P * G2);
#pragma omp parallel for schedule(static)
  for (int p = 0; p < P; ++p) {
    const float* hp = h + (size_t)p * O1;
    for (int j = 0; j < C2; ++j) {
      const float g0 = hp[2 * j], g1 = hp[2 * j + 1];
      ae[(size_t)p * C2 + j] = g0 / (1.0f + expf(-g0)) * hp[I + 2 * j];
      ao[(size_t)p * C2 + j] = g1 / (1.0f + expf(-g1)) * hp[I + 2 * j + 1];
    }
    for (int g = 0; g < G2; ++g) {
      float a = 0.f;
      for (int j = g * half; j < (g + 1) * half; ++j) a += ae[(size_t)p * C2 + j] + ao[(size_t)p * C2 + j];
      asum[(size_t)p * G2 + g] = a;
    }
  }
  float* y = (float*)malloc(sizeof(float) * (size_t)P * H);
#pragma omp parallel for schedule(static)
  for (long t = 0; t < (long)k * H; ++t) {
    const int e = (int)(t / H), o = (int)(t - (long)e * H);
    const uint8_t* raw = (const uint8_t*)(uintptr_t)ptrs[4 * e + 2] + (size_t)o * C2;
    const float* sc = (const float*)(uintptr_t)ptrs[4 * e + 3] + (size_t)o * G2;
    const int xr = xors[e];
    for (int64_t p = poff[e]; p < poff[e + 1]; ++p) {
      float acc = 0.f, corr = 0.f;
      for (int g = 0; g < G2; ++g) {
        float part = 0.f;
        const int b0 = g * half;
        for (int j = 0; j < half; ++j) {
          const int b = raw[b0 + j] ^ xr;
          part += (float)(b & 15) * ae[p * C2 + b0 + j] + (float)(b >> 4) * ao[p * C2 + b0 + j];
        }
        acc += part * sc[g];
        corr += sc[g] * asum[p * G2 + g];
      }
      y[(size_t)p * H + o] = acc - 8.0f * corr;
    }
  }
  for (int p = 0; p < P; ++p) {
    float* dst = out + (size_t)prow[p] * H;
    const float w = pw[p];
    for (int j = 0; j < H; ++j) dst[j] += w * y[(size_t)p * H + j];
  }
  free(xe);
  free(xo);
  free(xsum);
  free(h);
  free(ae);
  free(ao);
  free(asum);
  free(y);
}

/* _f16, moelan/kernels.py:244-255 */
static float f16(uint8_t lo, uint8_t hi) {
  const int h = lo | (hi << 8);
  const int e = (h >> 10) & 0x1F, m = h & 0x3FF;
  float v;
  if (e == 0) v = (float)m * 5.9604644775390625e-08f;
  else if (e == 31) v = INFINITY;
  else v = ldexpf((float)(1024 + m), e - 25);
  return (h & 0x8000) ? -v : v;
}

/* _mv_q8_0, moelan/kernels.py:482-497 */
void ref_mv_q8_0(const float* x, int n, const uint8_t* raw, int O, int cols, float* y) {
  const int nb = cols / 32;
#pragma omp parallel for schedule(static)
  for (int o = 0; o < O; ++o) {
    const uint8_t* row = raw + (size_t)o * nb * 34;
    for (int r = 0; r < n; ++r) {
      float acc = 0.f;
      for (int b = 0; b < nb; ++b) {
        const uint8_t* p = row + b * 34;
        float s = 0.f;
        for (int j = 0; j < 32; ++j) s += (float)(int8_t)p[2 + j] * x[(size_t)r * cols + b * 32 + j];
        acc += f16(p[0], p[1]) * s;
      }
      y[(size_t)r * O + o] = acc;
    }
  }
}

/* _scale_min_k4, moelan/kernels.py:310-316 */
static void scale_min(int j, const uint8_t* s, int* sc, int* m) {
  if (j < 4) {
    *sc = s[j] & 63;
    *m = s[j + 4] & 63;
  } else {
    *sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
    *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
  }
}

/* _mv_q4_k, moelan/kernels.py:499-527 (x sums per 32 as gguf_matmul_t :988) */
void ref_mv_q4_k(const float* x, int n, const uint8_t* raw, int O, int cols, float* y) {
  const int nb = cols / 256, ng = cols / 32;
  float* xs = (float*)malloc(sizeof(float) * (size_t)n * ng);
  for (int r = 0; r < n; ++r)
    for (int g = 0; g < ng; ++g) {
      float a = 0.f;
      for (int j = 0; j < 32; ++j) a += x[(size_t)r * cols + g * 32 + j];
      xs[(size_t)r * ng + g] = a;
    }
#pragma omp parallel for schedule(static)
  for (int o = 0; o < O; ++o) {
    const uint8_t* row = raw + (size_t)o * nb * 144;
    for (int r = 0; r < n; ++r) {
      float acc = 0.f;
      for (int b = 0; b < nb; ++b) {
        const uint8_t* p = row + b * 144;
        const float d = f16(p[0], p[1]), dmin = f16(p[2], p[3]);
        for (int kk = 0; kk < 4; ++kk) {
          int sc1, m1, sc2, m2;
          scale_min(2 * kk, p + 4, &sc1, &m1);
          scale_min(2 * kk + 1, p + 4, &sc2, &m2);
          const uint8_t* q = p + 16 + kk * 32;
          const int x0 = b * 256 + kk * 64;
          float s1 = 0.f, s2 = 0.f;
          for (int l = 0; l < 32; ++l) {
            const int v = q[l];
            s1 += (float)(v & 15) * x[(size_t)r * cols + x0 + l];
            s2 += (float)(v >> 4) * x[(size_t)r * cols + x0 + 32 + l];
          }
          const int g = x0 / 32;
          acc += d * ((float)sc1 * s1 + (float)sc2 * s2) -
                 dmin * ((float)m1 * xs[(size_t)r * ng + g] + (float)m2 * xs[(size_t)r * ng + g + 1]);
        }
      }
      y[(size_t)r * O + o] = acc;
    }
  }
  free(xs);
}

/* threads an OpenMP parallel region uses here */
int ref_threads(void) { return omp_get_max_threads(); }
