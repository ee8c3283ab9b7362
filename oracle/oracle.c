/*
 * CPU oracle for the full-attention hot path -- TEST INFRASTRUCTURE ONLY.
 *
 * Loaded by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg as
 * the checker; never by the product library. Built with -O2 -ffp-contract=off
 * -fno-fast-math so that every f32 statement rounds exactly once, like the
 * reference's host mirror of the quantizers.
 *
 * Pinning (what checks each function besides its own formula):
 *   orc_f32_to_f16 / orc_f16_to_f32  exhaustive vs numpy float16 casts and, when
 *                                    built, the reference's own fp16.h (oracle/_ref)
 *   orc_store_rows                   golden vectors (tests/golden), closed forms
 *                                    (zero block, constant block, ties, .5 cases),
 *                                    round-trip error bound in quant steps
 *   orc_load_rows                    closed forms per type (d*q, d*(n-8), ...)
 *   orc_attn_*                       1 key -> V, identical keys -> mean(V),
 *                                    brute-force numpy softmax on small cases
 *   orc_merge                        equality with unsplit attention
 *   orc_sigmoid_gate                 closed form vs numpy
 *   orc_rms_norm                     power-of-two rows (exact scale), f64 numpy
 *                                    formula, the halving tree vs a plain sum
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 --- */

/* IEEE half -> float. Follows the device conversion the reference kernels use
 * (fp16.h:16-19, V_CVT_F32_F16), so inf/NaN decode as inf/NaN. */
float orc_f16_to_f32(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e = (h >> 10) & 0x1fu;
  const uint32_t m = h & 0x3ffu;
  float f;
  if (e == 0) {
    f = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
    return sign ? -f : f;
  }
  uint32_t bits;
  if (e == 31)
    bits = sign | 0x7f800000u | (m << 13);
  else
    bits = sign | ((e + 112u) << 23) | (m << 13);
  memcpy(&f, &bits, 4);
  return f;
}

/* float -> half, round to nearest even (fp16.h:36-57). Overflow, inf and NaN
 * all give a signed infinity; magnitudes below half the smallest subnormal
 * give a signed zero. */
uint16_t orc_f32_to_f16(float f) {
  uint32_t x;
  memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t a = x & 0x7fffffffu;
  const int e = (int)(a >> 23) - 112; /* biased half exponent */
  if (e >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return (uint16_t)sign;
    const uint32_t m = (a & 0x7fffffu) | 0x800000u;
    const int sh = 14 - e;
    uint32_t r = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u);
    const uint32_t half = 1u << (sh - 1);
    if (rem > half || (rem == half && (r & 1u))) ++r;
    return (uint16_t)(sign | r);
  }
  uint32_t r = ((uint32_t)e << 10) | ((a >> 13) & 0x3ffu);
  const uint32_t rem = a & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (r & 1u))) ++r; /* carry may reach inf: correct */
  return (uint16_t)(sign | r);
}

/* --------------------------------------------------------------- tables --- */

enum { T_F32 = 0, T_F16 = 1, T_Q8_0 = 2, T_Q4_0 = 3, T_Q5_0 = 4, T_Q4_1 = 5 };

/* Block sizes in bytes per 32 elements (llama.cpp layouts, quants.h:88-101 and
 * kv.h:75-87): q8_0 {f16 d; i8 qs[32]} = 34, q4_0 {f16 d; u8 qs[16]} = 18,
 * q5_0 {f16 d; u8 qh[4]; u8 qs[16]} = 22, q4_1 {f16 d; f16 m; u8 qs[16]} = 20. */
static int block_bytes(int type) {
  switch (type) {
    case T_Q8_0: return 34;
    case T_Q4_0: return 18;
    case T_Q5_0: return 22;
    case T_Q4_1: return 20;
    default: return 0;
  }
}

int64_t orc_row_bytes(int type, int head_dim) {
  const int64_t blocks = ((int64_t)head_dim + 31) / 32;
  switch (type) {
    case T_F32: return (int64_t)head_dim * 4;
    case T_F16: return (int64_t)head_dim * 2;
    case T_Q8_0:
    case T_Q4_0:
    case T_Q5_0:
    case T_Q4_1: return blocks * block_bytes(type);
    default: return -1;
  }
}

double orc_bytes_per_elem(int type) {
  switch (type) {
    case T_F32: return 4.0;
    case T_F16: return 2.0;
    case T_Q8_0:
    case T_Q4_0:
    case T_Q5_0:
    case T_Q4_1: return block_bytes(type) / 32.0;
    default: return 0.0;
  }
}

static void put_u16(uint8_t *p, uint16_t v) {
  p[0] = (uint8_t)(v & 0xffu);
  p[1] = (uint8_t)(v >> 8);
}
static uint16_t get_u16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* (int8_t) conversion of a float, then clamp to [0, hi]: the quantizers'
 * `(int)(std::int8_t)(x + c)` followed by MIN/MAX (kv.h:429-432,460-463,492-495).
 * C's float->int8 conversion truncates toward zero; values outside int8 are
 * undefined in C, and the kernels only ever produce in-range values here
 * (|x*id| <= 16, 8 or 15 by construction, plus the constant). */
static int trunc_clamp(float x, int hi) {
  int q = (int)(int8_t)(int)x;
  if (q > hi) q = hi;
  if (q < 0) q = 0;
  return q;
}

/* q8_0 (kv.h:402-411): d = amax/127, qs = round(x/d) half away from zero. */
static void quant_q8_0(const float *x, uint8_t *y) {
  float amax = 0.0f;
  for (int j = 0; j < 32; ++j) amax = fmaxf(amax, fabsf(x[j]));
  const float d = amax / 127.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_u16(y, orc_f32_to_f16(d));
  for (int j = 0; j < 32; ++j) {
    const float s = x[j] * id;
    y[2 + j] = (uint8_t)(int8_t)roundf(s);
  }
}

/* signed value of largest magnitude, first occurrence wins on ties
 * (strict `amax < |v|`, kv.h:478-485). */
static float signed_absmax(const float *x) {
  float amax = 0.0f, vmax = 0.0f;
  for (int j = 0; j < 32; ++j) {
    if (amax < fabsf(x[j])) {
      amax = fabsf(x[j]);
      vmax = x[j];
    }
  }
  return vmax;
}

/* q4_0 (kv.h:476-499): d = vmax/-8, q = trunc(x/d + 8.5) clamped to [0,15];
 * byte j holds element j (low nibble) and j+16 (high nibble). */
static void quant_q4_0(const float *x, uint8_t *y) {
  const float d = signed_absmax(x) / -8.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_u16(y, orc_f32_to_f16(d));
  for (int j = 0; j < 16; ++j) {
    const float a = x[j] * id, b = x[j + 16] * id;
    const int q0 = trunc_clamp(a + 8.5f, 15), q1 = trunc_clamp(b + 8.5f, 15);
    y[2 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

/* q5_0 (kv.h:412-445): d = vmax/-16, q = trunc(x/d + 16.5) clamped to [0,31];
 * low 4 bits as q4_0's nibbles, bit 4 of element e into bit e of the
 * little-endian 32-bit qh plane. */
static void quant_q5_0(const float *x, uint8_t *y) {
  const float d = signed_absmax(x) / -16.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_u16(y, orc_f32_to_f16(d));
  uint32_t qh = 0;
  for (int j = 0; j < 16; ++j) {
    const float a = x[j] * id, b = x[j + 16] * id;
    const int q0 = trunc_clamp(a + 16.5f, 31), q1 = trunc_clamp(b + 16.5f, 31);
    y[6 + j] = (uint8_t)((q0 & 15) | ((q1 & 15) << 4));
    qh |= (uint32_t)(q0 >> 4) << j;
    qh |= (uint32_t)(q1 >> 4) << (j + 16);
  }
  for (int i = 0; i < 4; ++i) y[2 + i] = (uint8_t)(qh >> (8 * i));
}

/* q4_1 (kv.h:446-467): d = (max-min)/15, m = min, q = trunc((x-min)/d + 0.5)
 * clamped to [0,15]. */
static void quant_q4_1(const float *x, uint8_t *y) {
  float lo = x[0], hi = x[0];
  for (int j = 1; j < 32; ++j) {
    lo = fminf(lo, x[j]);
    hi = fmaxf(hi, x[j]);
  }
  const float d = (hi - lo) / 15.0f;
  const float id = d != 0.0f ? 1.0f / d : 0.0f;
  put_u16(y, orc_f32_to_f16(d));
  put_u16(y + 2, orc_f32_to_f16(lo));
  for (int j = 0; j < 16; ++j) {
    const float a = (x[j] - lo) * id, b = (x[j + 16] - lo) * id;
    const int q0 = trunc_clamp(a + 0.5f, 15), q1 = trunc_clamp(b + 0.5f, 15);
    y[4 + j] = (uint8_t)(q0 | (q1 << 4));
  }
}

int orc_store_rows(int type, const float *src, void *dst, int64_t width) {
  uint8_t *out = (uint8_t *)dst;
  if (width < 0) return -1;
  switch (type) {
    case T_F32: memcpy(out, src, (size_t)width * 4); return 0;
    case T_F16:
      for (int64_t i = 0; i < width; ++i) put_u16(out + 2 * i, orc_f32_to_f16(src[i]));
      return 0;
    case T_Q8_0:
    case T_Q4_0:
    case T_Q5_0:
    case T_Q4_1: break;
    default: return -1;
  }
  if (width % 32) return -1;
  const int bb = block_bytes(type);
  for (int64_t b = 0; b < width / 32; ++b) {
    const float *x = src + b * 32;
    uint8_t *y = out + b * bb;
    if (type == T_Q8_0) quant_q8_0(x, y);
    else if (type == T_Q4_0) quant_q4_0(x, y);
    else if (type == T_Q5_0) quant_q5_0(x, y);
    else quant_q4_1(x, y);
  }
  return 0;
}

/* Dequantize one 32-element block (kv.h:177-229). Every product below is exact
 * in f32 (11-bit d times a <= 8-bit integer), so the value is unique. */
static void dequant_block(int type, const uint8_t *y, float *x) {
  const float d = orc_f16_to_f32(get_u16(y));
  for (int j = 0; j < 32; ++j) {
    const int i = j & 15;
    switch (type) {
      case T_Q8_0: x[j] = d * (float)(int8_t)y[2 + j]; break;
      case T_Q4_0: {
        const int n = j < 16 ? (y[2 + i] & 15) : (y[2 + i] >> 4);
        x[j] = d * (float)(n - 8);
        break;
      }
      case T_Q5_0: {
        const int n = j < 16 ? (y[6 + i] & 15) : (y[6 + i] >> 4);
        const int h = (y[2 + (j >> 3)] >> (j & 7)) & 1;
        x[j] = d * (float)((n | (h << 4)) - 16);
        break;
      }
      default: { /* q4_1: d*q + m, two roundings (kv.h:228) */
        const float m = orc_f16_to_f32(get_u16(y + 2));
        const int n = j < 16 ? (y[4 + i] & 15) : (y[4 + i] >> 4);
        const float p = d * (float)n;
        x[j] = p + m;
        break;
      }
    }
  }
}

int orc_load_rows(int type, const void *src, float *dst, int64_t width) {
  const uint8_t *in = (const uint8_t *)src;
  if (width < 0) return -1;
  switch (type) {
    case T_F32: memcpy(dst, in, (size_t)width * 4); return 0;
    case T_F16:
      for (int64_t i = 0; i < width; ++i) dst[i] = orc_f16_to_f32(get_u16(in + 2 * i));
      return 0;
    case T_Q8_0:
    case T_Q4_0:
    case T_Q5_0:
    case T_Q4_1: break;
    default: return -1;
  }
  if (width % 32) return -1;
  const int bb = block_bytes(type);
  for (int64_t b = 0; b < width / 32; ++b) dequant_block(type, in + b * bb, dst + b * 32);
  return 0;
}

/* ----------------------------------------------------------------- fill --- */

/* kv.h:508-513: multiplicative hash, top 24 bits mapped to [-1, 1). */
float orc_kv_rand(uint32_t idx, uint32_t seed) {
  uint32_t h = (idx * 2654435761u) ^ (seed * 2246822519u);
  h ^= h >> 13;
  h *= 1274126177u;
  return (float)(h >> 8) / 8388608.0f - 1.0f;
}

int orc_fill(int type, void *dst, int64_t n_rows, int head_dim, uint32_t seed) {
  const int64_t rb = orc_row_bytes(type, head_dim);
  if (rb <= 0 || head_dim % 32) return -1;
  float *row = (float *)malloc((size_t)head_dim * sizeof(float));
  if (!row) return -1;
  for (int64_t r = 0; r < n_rows; ++r) {
    for (int e = 0; e < head_dim; ++e) row[e] = orc_kv_rand((uint32_t)(r * head_dim + e), seed);
    orc_store_rows(type, row, (uint8_t *)dst + r * rb, head_dim);
  }
  free(row);
  return 0;
}

/* ------------------------------------------------------------ attention --- */

/* One query head against keys 0..t of its kv head. K and V rows of that kv
 * head have been dequantized into kd/vd ([t+1][hd] f32). Double softmax with
 * the max subtracted, as check_rope_gpu.hip:113-128. */
static void attend_one(const float *qh, const float *kd, const float *vd, int t, int hd,
                       double scale, double *sc, double *acc, float *out) {
  if (t < 0) {
    for (int i = 0; i < hd; ++i) out[i] = 0.0f;
    return;
  }
  double m = -INFINITY;
  for (int j = 0; j <= t; ++j) {
    const float *kr = kd + (int64_t)j * hd;
    double s = 0.0;
    for (int i = 0; i < hd; ++i) s += (double)qh[i] * (double)kr[i];
    sc[j] = s * scale;
    if (sc[j] > m) m = sc[j];
  }
  double sum = 0.0;
  for (int j = 0; j <= t; ++j) {
    sc[j] = exp(sc[j] - m);
    sum += sc[j];
  }
  for (int i = 0; i < hd; ++i) acc[i] = 0.0;
  for (int j = 0; j <= t; ++j) {
    const double w = sc[j] / sum;
    const float *vr = vd + (int64_t)j * hd;
    for (int i = 0; i < hd; ++i) acc[i] += w * (double)vr[i];
  }
  for (int i = 0; i < hd; ++i) out[i] = (float)acc[i];
}

/* Dequantize rows 0..n-1 of kv head kvh from a [pos][n_kv][row] cache. */
static int gather_rows(int type, const void *cache, int n, int n_kv, int kvh, int hd, float *dst) {
  const int64_t rb = orc_row_bytes(type, hd);
  if (rb <= 0) return -1;
  for (int j = 0; j < n; ++j) {
    const uint8_t *row = (const uint8_t *)cache + ((int64_t)j * n_kv + kvh) * rb;
    if (orc_load_rows(type, row, dst + (int64_t)j * hd, hd)) return -1;
  }
  return 0;
}

int orc_attn_batch(const float *q, const void *k, const void *v, float *out, const int *pos,
                   int n_tok, int n_head, int n_head_kv, int head_dim, float scale, int kt, int vt,
                   int n_threads) {
  if (n_head_kv <= 0 || n_head % n_head_kv || head_dim <= 0 || head_dim % 32) return -1;
  if (orc_row_bytes(kt, head_dim) <= 0 || orc_row_bytes(vt, head_dim) <= 0) return -1;
  int tmax = -1;
  for (int i = 0; i < n_tok; ++i)
    if (pos[i] > tmax) tmax = pos[i];
  const int n = tmax + 1;
  const int grp = n_head / n_head_kv;
  float *kd = (float *)malloc(((size_t)(n > 0 ? n : 1)) * head_dim * sizeof(float));
  float *vd = (float *)malloc(((size_t)(n > 0 ? n : 1)) * head_dim * sizeof(float));
  int rc = (kd && vd) ? 0 : -1;
  if (n_threads < 1) n_threads = 1;
  for (int kvh = 0; kvh < n_head_kv && rc == 0; ++kvh) {
    if (gather_rows(kt, k, n, n_head_kv, kvh, head_dim, kd) ||
        gather_rows(vt, v, n, n_head_kv, kvh, head_dim, vd)) {
      rc = -1;
      break;
    }
    const int items = n_tok * grp;
#pragma omp parallel for num_threads(n_threads) schedule(dynamic, 1)
    for (int it = 0; it < items; ++it) {
      const int tok = it / grp;
      const int h = kvh * grp + it % grp;
      double *sc = (double *)malloc(((size_t)(n > 0 ? n : 1)) * sizeof(double));
      double *acc = (double *)malloc((size_t)head_dim * sizeof(double));
      const int64_t off = ((int64_t)tok * n_head + h) * head_dim;
      attend_one(q + off, kd, vd, pos[tok], head_dim, (double)scale, sc, acc, out + off);
      free(sc);
      free(acc);
    }
  }
  free(kd);
  free(vd);
  return rc;
}

int orc_attn_decode(const float *q, const void *k, const void *v, float *out, int t, int n_head,
                    int n_head_kv, int head_dim, float scale, int kt, int vt, int n_threads) {
  return orc_attn_batch(q, k, v, out, &t, 1, n_head, n_head_kv, head_dim, scale, kt, vt,
                        n_threads);
}

void orc_merge(const float *partial, float *out, int n_rows, int head_dim, int n_splits) {
  const int64_t rec = 2 + head_dim;
  for (int r = 0; r < n_rows; ++r) {
    const float *base = partial + (int64_t)r * n_splits * rec;
    double mm = -INFINITY;
    for (int s = 0; s < n_splits; ++s)
      if ((double)base[s * rec] > mm) mm = base[s * rec];
    float *o = out + (int64_t)r * head_dim;
    if (mm == -INFINITY) {
      for (int i = 0; i < head_dim; ++i) o[i] = 0.0f;
      continue;
    }
    double l = 0.0;
    for (int s = 0; s < n_splits; ++s) {
      const double m = base[s * rec];
      if (m != -INFINITY) l += (double)base[s * rec + 1] * exp(m - mm);
    }
    for (int i = 0; i < head_dim; ++i) {
      double a = 0.0;
      for (int s = 0; s < n_splits; ++s) {
        const double m = base[s * rec];
        if (m != -INFINITY) a += (double)base[s * rec + 2 + i] * exp(m - mm);
      }
      o[i] = l > 0.0 ? (float)(a / l) : 0.0f;
    }
  }
}

void orc_sigmoid_gate(float *g, float *y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    const float e = expf(-g[i]);
    const float s = 1.0f / (1.0f + e);
    g[i] = s;
    y[i] = y[i] * s;
  }
}

void orc_rope(float *x, int n_tokens, int n_heads, int head_dim, int n_rot, float freq_base,
              const int *pos) {
  const int pairs = n_rot / 2;
  for (int t = 0; t < n_tokens; ++t)
    for (int h = 0; h < n_heads; ++h) {
      float *b = x + ((int64_t)t * n_heads + h) * head_dim;
      for (int p = 0; p < pairs; ++p) {
        /* the angle is formed in f32 like attn.cuh:39; cos/sin then in double */
        const float thf = (float)pos[t] * powf(freq_base, -2.0f * (float)p / (float)n_rot);
        const double th = (double)thf;
        const double c = cos(th), s = sin(th);
        const double x0 = b[p], x1 = b[p + pairs];
        b[p] = (float)(x0 * c - x1 * s);
        b[p + pairs] = (float)(x0 * s + x1 * c);
      }
    }
}

void orc_rms_norm(const float *x, const float *w, float *y, int64_t nrows, int64_t ncols,
                  float eps) {
  enum { T = 256 };
  for (int64_t r = 0; r < nrows; ++r) {
    const float *xr = x + r * ncols;
    float *yr = y + r * ncols;
    float part[T];
    for (int t = 0; t < T; ++t) {
      float acc = 0.0f;
      for (int64_t i = t; i < ncols; i += T) acc = fmaf(xr[i], xr[i], acc);
      part[t] = acc;
    }
    for (int s = T / 2; s > 0; s >>= 1)
      for (int t = 0; t < s; ++t) part[t] = part[t] + part[t + s];
    const float mean = part[0] / (float)ncols + eps;
    const float scale = (float)(1.0 / sqrt((double)mean));
    for (int64_t i = 0; i < ncols; ++i) {
      const float v = xr[i] * scale;
      yr[i] = w ? v * w[i] : v;
    }
  }
}

/* ------------------------------------------------------------- inputs --- */

static uint64_t splitmix64(uint64_t *s) {
  uint64_t z = (*s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

void orc_randn(float *dst, int64_t n, uint64_t seed) {
  uint64_t s = seed;
  for (int64_t i = 0; i < n; i += 2) {
    /* two uniforms in (0,1] from the top 53 bits */
    const double u1 = ((double)(splitmix64(&s) >> 11) + 1.0) * (1.0 / 9007199254740992.0);
    const double u2 = (double)(splitmix64(&s) >> 11) * (1.0 / 9007199254740992.0);
    const double r = sqrt(-2.0 * log(u1));
    const double a = 6.283185307179586 * u2;
    dst[i] = (float)(r * cos(a));
    if (i + 1 < n) dst[i + 1] = (float)(r * sin(a));
  }
}
