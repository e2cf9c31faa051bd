/*
 * CPU oracle for the causal GQA attention path — TEST INFRASTRUCTURE ONLY.
 * The checker, never the product: only tests/, smoke() and bench.py's
 * cpu_baseline leg may load it. See attn_oracle.h for the contract of each
 * function and the reference lines it restates.
 *
 * Build flags matter: -ffp-contract=off keeps every f32 multiply and add a
 * separately rounded IEEE operation (the reference kernel's source order),
 * and -fno-fast-math keeps the summation order exactly as written.
 */
#include "attn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- f16 -- */

uint16_t orc_f32_to_f16(float value) {
  uint32_t x;
  memcpy(&x, &value, sizeof x);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t exponent = (x >> 23) & 0xffu;
  uint32_t mantissa = x & 0x7fffffu;
  if (exponent == 0xffu) {
    if (mantissa != 0) /* NaN: keep it quiet and non-zero */
      return (uint16_t)(sign | 0x7e00u | (mantissa >> 13));
    return (uint16_t)(sign | 0x7c00u);
  }
  if (exponent == 0) /* f32 zero or subnormal: far below the f16 range */
    return (uint16_t)sign;
  int32_t e = (int32_t)exponent - 127 + 15;
  if (e >= 31)
    return (uint16_t)(sign | 0x7c00u);
  if (e >= 1) {
    uint32_t h = ((uint32_t)e << 10) | (mantissa >> 13);
    uint32_t rem = mantissa & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u)))
      h += 1; /* a carry into the exponent is the correct rounding */
    return (uint16_t)(sign | h);
  }
  /* f16 subnormal: value = full * 2^(exponent - 150), unit 2^-24. */
  uint32_t full = mantissa | 0x800000u;
  uint32_t shift = (uint32_t)(126 - (int32_t)exponent);
  if (shift >= 25)
    return (uint16_t)sign;
  uint32_t h = full >> shift;
  uint32_t rem = full & ((1u << shift) - 1u);
  uint32_t half = 1u << (shift - 1);
  if (rem > half || (rem == half && (h & 1u)))
    h += 1;
  return (uint16_t)(sign | h);
}

float orc_f16_to_f32(uint16_t bits) {
  uint32_t sign = ((uint32_t)bits & 0x8000u) << 16;
  uint32_t exponent = ((uint32_t)bits >> 10) & 0x1fu;
  uint32_t mantissa = (uint32_t)bits & 0x3ffu;
  uint32_t x;
  if (exponent == 0x1fu) {
    x = sign | 0x7f800000u | (mantissa << 13);
  } else if (exponent != 0) {
    x = sign | ((exponent - 15 + 127) << 23) | (mantissa << 13);
  } else if (mantissa == 0) {
    x = sign;
  } else {
    /* subnormal: normalise */
    uint32_t e = 127 - 15 + 1;
    while ((mantissa & 0x400u) == 0) {
      mantissa <<= 1;
      e -= 1;
    }
    x = sign | (e << 23) | ((mantissa & 0x3ffu) << 13);
  }
  float f;
  memcpy(&f, &x, sizeof f);
  return f;
}

void orc_f32_to_f16_array(const float *src, uint16_t *dst, size_t n) {
  for (size_t i = 0; i < n; ++i)
    dst[i] = orc_f32_to_f16(src[i]);
}

void orc_f16_to_f32_array(const uint16_t *src, float *dst, size_t n) {
  for (size_t i = 0; i < n; ++i)
    dst[i] = orc_f16_to_f32(src[i]);
}

/* ---------------------------------------------------------- XorShift64 -- */

uint64_t orc_xorshift_seed(uint64_t seed) {
  /* qwen3.rs:1016-1023: a zero seed is replaced by the golden-ratio word. */
  return seed == 0 ? 0x9e3779b97f4a7c15ull : seed;
}

static uint64_t xorshift_step(uint64_t value) {
  value ^= value << 13;
  value ^= value >> 7;
  value ^= value << 17;
  return value;
}

double orc_xorshift_next_f64(uint64_t *state) {
  /* qwen3.rs:1025-1032: value / (u64::MAX as f64 + 1.0) == value / 2^64 */
  uint64_t value = xorshift_step(*state);
  *state = value;
  return (double)value / 18446744073709551616.0;
}

/* The step is linear over GF(2)^64; a map is stored as its 64 column images. */
typedef struct {
  uint64_t column[64];
} gf2_map;

static uint64_t gf2_apply(const gf2_map *map, uint64_t x) {
  uint64_t y = 0;
  for (int bit = 0; bit < 64; ++bit)
    if ((x >> bit) & 1u)
      y ^= map->column[bit];
  return y;
}

static void gf2_compose(const gf2_map *outer, const gf2_map *inner,
                        gf2_map *result) {
  gf2_map tmp;
  for (int bit = 0; bit < 64; ++bit)
    tmp.column[bit] = gf2_apply(outer, inner->column[bit]);
  *result = tmp;
}

uint64_t orc_xorshift_jump(uint64_t state, uint64_t steps) {
  gf2_map power;
  for (int bit = 0; bit < 64; ++bit)
    power.column[bit] = xorshift_step(1ull << bit);
  while (steps != 0) {
    if (steps & 1u)
      state = gf2_apply(&power, state);
    gf2_compose(&power, &power, &power);
    steps >>= 1;
  }
  return state;
}

static uint16_t normal_from_state(uint64_t *state) {
  double u1 = orc_xorshift_next_f64(state);
  double u2 = orc_xorshift_next_f64(state);
  double radius = sqrt(-2.0 * log(1.0 - u1));
  double z = radius * cos(2.0 * M_PI * u2);
  return orc_f32_to_f16((float)z);
}

void orc_fill_normal_f16(uint64_t seed, uint16_t *out, size_t n, int threads) {
  uint64_t start = orc_xorshift_seed(seed);
  if (threads < 1)
    threads = 1;
  if ((size_t)threads > n / 65536 + 1)
    threads = (int)(n / 65536 + 1);
#pragma omp parallel for num_threads(threads) schedule(static, 1)
  for (int chunk = 0; chunk < threads; ++chunk) {
    size_t begin = n * (size_t)chunk / (size_t)threads;
    size_t end = n * (size_t)(chunk + 1) / (size_t)threads;
    uint64_t state = orc_xorshift_jump(start, 2 * (uint64_t)begin);
    for (size_t i = begin; i < end; ++i)
      out[i] = normal_from_state(&state);
  }
}

void orc_fill_uniform_u32(uint64_t seed, uint32_t lo, uint32_t hi,
                          uint32_t *out, size_t n) {
  uint64_t state = orc_xorshift_seed(seed);
  double span = (double)hi - (double)lo + 1.0;
  for (size_t i = 0; i < n; ++i) {
    double u = orc_xorshift_next_f64(&state);
    double value = floor(u * span);
    uint32_t offset = value >= span ? hi - lo : (uint32_t)value;
    out[i] = lo + offset;
  }
}

/* ----------------------------------------------------------- attention -- */

static int64_t elem(const int64_t stride[3], uint32_t a, uint32_t b,
                    uint32_t c) {
  return (int64_t)a * stride[0] + (int64_t)b * stride[1] +
         (int64_t)c * stride[2];
}

int orc_attention(const orc_attention_args *a) {
  if (a == NULL || a->q_heads == 0 || a->kv_heads == 0 || a->head_dim == 0 ||
      a->q_heads % a->kv_heads != 0)
    return -1;
  const uint32_t T = a->tokens, Hq = a->q_heads, Hkv = a->kv_heads;
  const uint32_t D = a->head_dim, L = a->kv_length;
  const uint32_t group = Hq / Hkv;
  const uint32_t n_rows = a->rows != NULL ? a->n_rows : T;
  for (uint32_t r = 0; a->rows != NULL && r < n_rows; ++r)
    if (a->rows[r] >= T)
      return -1;

  /* K transposed to [Hkv][D][L] and V to [Hkv][L][D], both as f32 (exact). */
  size_t kv_elems = (size_t)Hkv * L * D;
  float *kt = malloc(kv_elems * sizeof(float) + 1);
  float *vf = malloc(kv_elems * sizeof(float) + 1);
  double *kt64 = NULL, *vf64 = NULL;
  if (a->out_f64 != NULL) {
    kt64 = malloc(kv_elems * sizeof(double) + 1);
    vf64 = malloc(kv_elems * sizeof(double) + 1);
  }
  if (kt == NULL || vf == NULL || (a->out_f64 != NULL && (!kt64 || !vf64))) {
    free(kt), free(vf), free(kt64), free(vf64);
    return -1;
  }
  int threads = a->threads < 1 ? 1 : a->threads;
#pragma omp parallel for num_threads(threads) collapse(2) schedule(static)
  for (uint32_t h = 0; h < Hkv; ++h)
    for (uint32_t j = 0; j < L; ++j)
      for (uint32_t x = 0; x < D; ++x) {
        float kv = orc_f16_to_f32(a->k[elem(a->k_stride, j, h, x)]);
        float vv = orc_f16_to_f32(a->v[elem(a->v_stride, j, h, x)]);
        kt[((size_t)h * D + x) * L + j] = kv;
        vf[((size_t)h * L + j) * D + x] = vv;
        if (kt64 != NULL) {
          kt64[((size_t)h * D + x) * L + j] = kv;
          vf64[((size_t)h * L + j) * D + x] = vv;
        }
      }

  /* transformer.metal:1592: scale = rsqrt(float(head_dim)), applied after
   * the dot product (:1598). */
  const float scale = 1.0f / sqrtf((float)D);
  const double scale64 = 1.0 / sqrt((double)D);

#pragma omp parallel num_threads(threads)
  {
    float *q = malloc(sizeof(float) * D);
    float *score = malloc(sizeof(float) * (L + 1));
    float *num = malloc(sizeof(float) * D);
    double *q64 = malloc(sizeof(double) * D);
    double *score64 = malloc(sizeof(double) * (L + 1));
    double *num64 = malloc(sizeof(double) * D);
#pragma omp for collapse(2) schedule(dynamic, 4)
    for (uint32_t r = 0; r < n_rows; ++r)
      for (uint32_t h = 0; h < Hq; ++h) {
        uint32_t qi = a->rows != NULL ? a->rows[r] : r;
        uint32_t kvh = h / group;
        /* transformer.metal:1589-1590 */
        uint64_t window = (uint64_t)a->query_offset + qi + 1;
        uint32_t available =
            a->causal != 0 ? (window < L ? (uint32_t)window : L) : L;
        for (uint32_t x = 0; x < D; ++x)
          q[x] = orc_f16_to_f32(a->q[elem(a->q_stride, qi, h, x)]);
        const float *khead = kt + (size_t)kvh * D * L;
        const float *vhead = vf + (size_t)kvh * L * D;
        /* Scores summed over x in ascending order (:1594-1597), each key's
         * chain independent, so the loop over j vectorises exactly. */
        for (uint32_t j = 0; j < available; ++j)
          score[j] = 0.0f;
        for (uint32_t x = 0; x < D; ++x) {
          const float qx = q[x];
          const float *krow = khead + (size_t)x * L;
          for (uint32_t j = 0; j < available; ++j)
            score[j] += qx * krow[j];
        }
        /* Pass 1: maximum of score * scale (:1593-1599). */
        float maximum = -INFINITY;
        for (uint32_t j = 0; j < available; ++j) {
          float s = score[j] * scale;
          maximum = s > maximum ? s : maximum;
        }
        /* Pass 2: denominator and numerator, keys ascending (:1600-1610). */
        float denominator = 0.0f;
        for (uint32_t x = 0; x < D; ++x)
          num[x] = 0.0f;
        for (uint32_t j = 0; j < available; ++j) {
          float p = expf(score[j] * scale - maximum);
          denominator += p;
          const float *vrow = vhead + (size_t)j * D;
          for (uint32_t x = 0; x < D; ++x)
            num[x] += p * vrow[x];
        }
        size_t out_base = ((size_t)r * Hq + h) * D;
        for (uint32_t x = 0; x < D; ++x) {
          float o = num[x] / denominator; /* (:1611) */
          if (a->out_f32 != NULL)
            a->out_f32[out_base + x] = o;
          if (a->out_f16 != NULL)
            a->out_f16[out_base + x] = orc_f32_to_f16(o);
        }
        if (a->out_f64 != NULL) {
          const double *khead64 = kt64 + (size_t)kvh * D * L;
          const double *vhead64 = vf64 + (size_t)kvh * L * D;
          for (uint32_t x = 0; x < D; ++x)
            q64[x] = q[x];
          for (uint32_t j = 0; j < available; ++j)
            score64[j] = 0.0;
          for (uint32_t x = 0; x < D; ++x) {
            const double qx = q64[x];
            const double *krow = khead64 + (size_t)x * L;
            for (uint32_t j = 0; j < available; ++j)
              score64[j] += qx * krow[j];
          }
          double max64 = -INFINITY;
          for (uint32_t j = 0; j < available; ++j) {
            double s = score64[j] * scale64;
            max64 = s > max64 ? s : max64;
          }
          double den64 = 0.0;
          for (uint32_t x = 0; x < D; ++x)
            num64[x] = 0.0;
          for (uint32_t j = 0; j < available; ++j) {
            double p = exp(score64[j] * scale64 - max64);
            den64 += p;
            const double *vrow = vhead64 + (size_t)j * D;
            for (uint32_t x = 0; x < D; ++x)
              num64[x] += p * vrow[x];
          }
          for (uint32_t x = 0; x < D; ++x)
            a->out_f64[out_base + x] = num64[x] / den64;
        }
      }
    free(q), free(score), free(num), free(q64), free(score64), free(num64);
  }
  free(kt), free(vf), free(kt64), free(vf64);
  return 0;
}

/* ----------------------------------------------------- QK norm + RoPE -- */

int orc_qk_norm_rope(const uint16_t *q, const uint16_t *k, const uint16_t *q_w,
                     const uint16_t *k_w, uint32_t tokens, uint32_t q_heads,
                     uint32_t kv_heads, uint32_t head_dim, uint32_t offset,
                     float theta, float epsilon, uint16_t *q_out,
                     uint16_t *key_out) {
  if (head_dim == 0 || head_dim % 2 != 0)
    return -1;
  const uint32_t D = head_dim, half = head_dim / 2;
  uint32_t rows = tokens * (q_heads + kv_heads);
  for (uint32_t group = 0; group < rows; ++group) {
    /* transformer.metal:1543-1551: query rows first, then key rows. */
    uint32_t query_rows = tokens * q_heads;
    int is_query = group < query_rows;
    uint32_t row = is_query ? group : group - query_rows;
    uint32_t heads = is_query ? q_heads : kv_heads;
    uint32_t token = row / heads;
    const uint16_t *input = (is_query ? q : k) + (size_t)row * D;
    const uint16_t *weight = is_query ? q_w : k_w;
    uint16_t *output = (is_query ? q_out : key_out) + (size_t)row * D;
    /* :1552-1557 */
    float sum = 0.0f;
    for (uint32_t i = 0; i < D; ++i) {
      float value = orc_f16_to_f32(input[i]);
      sum += value * value;
    }
    float scale = 1.0f / sqrtf(sum / (float)D + epsilon);
    /* :1558-1575 */
    for (uint32_t pair = 0; pair < half; ++pair) {
      uint32_t second = pair + half;
      float x = orc_f16_to_f32(input[pair]) * scale *
                orc_f16_to_f32(weight[pair]);
      float y = orc_f16_to_f32(input[second]) * scale *
                orc_f16_to_f32(weight[second]);
      float frequency = powf(theta, -(float)(pair * 2) / (float)D);
      float angle = (float)(token + offset) * frequency;
      float c = cosf(angle), s = sinf(angle);
      output[pair] = orc_f32_to_f16(x * c - y * s);
      output[second] = orc_f32_to_f16(x * s + y * c);
    }
  }
  return 0;
}

/* ------------------------------------------------ attention neighbours -- */

int orc_rms_norm(const uint16_t *x, const uint16_t *w, uint64_t rows,
                 uint32_t width, float epsilon, uint16_t *out, float *out_f32) {
  if (width == 0)
    return -1;
  for (uint64_t row = 0; row < rows; ++row) {
    const uint16_t *in = x + row * width;
    /* transformer.metal:1330-1337 (one running sum instead of 32 lane sums
     * and a SIMD reduction: the same value up to f32 summation order). */
    float sum = 0.0f;
    for (uint32_t i = 0; i < width; ++i) {
      float value = orc_f16_to_f32(in[i]);
      sum += value * value;
    }
    float scale = 1.0f / sqrtf(sum / (float)width + epsilon);
    /* :1338-1339 */
    for (uint32_t i = 0; i < width; ++i) {
      float value = orc_f16_to_f32(in[i]) * scale * orc_f16_to_f32(w[i]);
      out[row * width + i] = orc_f32_to_f16(value);
      if (out_f32)
        out_f32[row * width + i] = value;
    }
  }
  return 0;
}

int orc_rope(const uint16_t *x, uint32_t tokens, uint32_t heads,
             uint32_t head_dim, uint32_t offset, float theta, uint16_t *out) {
  if (head_dim == 0 || head_dim % 2 != 0)
    return -1;
  const uint32_t half = head_dim / 2;
  for (uint32_t token = 0; token < tokens; ++token) {
    for (uint32_t head = 0; head < heads; ++head) {
      /* transformer.metal:1522-1530 */
      size_t base = ((size_t)token * heads + head) * head_dim;
      for (uint32_t pair = 0; pair < half; ++pair) {
        uint32_t second = pair + half;
        float frequency = powf(theta, -(float)(pair * 2) / (float)head_dim);
        float angle = (float)(token + offset) * frequency;
        float a = orc_f16_to_f32(x[base + pair]);
        float b = orc_f16_to_f32(x[base + second]);
        float c = cosf(angle), s = sinf(angle);
        out[base + pair] = orc_f32_to_f16(a * c - b * s);
        out[base + second] = orc_f32_to_f16(a * s + b * c);
      }
    }
  }
  return 0;
}

int orc_matmul(const uint16_t *x, const uint16_t *w, uint32_t m, uint32_t n,
               uint32_t k, uint16_t *out, float *out_f32, int threads) {
  if (threads <= 0)
    threads = omp_get_max_threads();
  /* transformer.metal:77-92: one f32 sum per output, k ascending. */
#pragma omp parallel for num_threads(threads) schedule(static)
  for (int64_t i = 0; i < (int64_t)m; ++i) {
    float *row = malloc(sizeof(float) * (size_t)k);
    if (row == NULL)
      abort();
    for (uint32_t c = 0; c < k; ++c)
      row[c] = orc_f16_to_f32(x[(size_t)i * k + c]);
    for (uint32_t j = 0; j < n; ++j) {
      const uint16_t *wr = w + (size_t)j * k;
      float sum = 0.0f;
      for (uint32_t c = 0; c < k; ++c)
        sum += row[c] * orc_f16_to_f32(wr[c]);
      out[(size_t)i * n + j] = orc_f32_to_f16(sum);
      if (out_f32)
        out_f32[(size_t)i * n + j] = sum;
    }
    free(row);
  }
  return 0;
}
