/*
 * CPU restatement of catena-models' Qwen3.5/3.6 token loop (test
 * infrastructure: the parity checker and the CPU baseline; never shipped or
 * called by the library). See oracle.h. Build with -ffp-contract=off so every
 * multiply and add rounds separately, as numeric.hex:10 specifies.
 *
 * Citations are file:line into hellas-ai/catena-models.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ------------------------------------------------------------------ bits */

static inline uint32_t fbits(float x) { uint32_t u; memcpy(&u, &x, 4); return u; }
static inline float bitsf(uint32_t u) { float x; memcpy(&x, &u, 4); return x; }

/* src/weights.rs:213-221: round-to-nearest-even, NaNs quieted. */
/* Planted mistakes (OX_PLANT_*, oracle.h): 0 in every normal use. The
 * pinning tests switch one on to show that their comparison with an
 * independent formulation fails for that mistake. */
static int g_plant = 0;
void ox_set_plant(int which) { g_plant = which; }

uint16_t ox_f2bf(float x) {
  uint32_t u = fbits(x);
  if (x != x) return (uint16_t)((u >> 16) | 0x0040u);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
float ox_bf2f(uint16_t b) { return bitsf((uint32_t)b << 16); }
static inline float rbf(float x) { return ox_bf2f(ox_f2bf(x)); }
/* bf16.add / bf16.mul (memory.hex:920-935): widen, operate in F32, round. */
static inline uint16_t bf_add(uint16_t a, uint16_t b) { return ox_f2bf(ox_bf2f(a) + ox_bf2f(b)); }
static inline uint16_t bf_mul(uint16_t a, uint16_t b) { return ox_f2bf(ox_bf2f(a) * ox_bf2f(b)); }

/* stdlib.math.round_to_u32 on a non-negative F32 (its catena-lang source is
 * not in the reference tree): nearest, ties away from zero. */
static inline uint32_t round_u32(float x) {
  float t = truncf(x);
  if (x - t >= 0.5f) t += 1.0f;
  return (uint32_t)t;
}

/* -------------------------------------------------------------- numerics */

/* numeric.hex:30-61 (stdlib.models.math.exp-scale). */
static float exp_scale(float y, uint32_t n, int negative) {
  uint32_t y_bits = fbits(y);
  uint32_t exponent = y_bits >> 23;
  int subnormal = exponent <= n;
  uint32_t shift = subnormal ? (n - exponent) + 1u : 1u;
  uint32_t fraction = y_bits % 0x00800000u;
  uint32_t significand = fraction + 0x00800000u;
  uint32_t truncated = significand >> shift;
  uint32_t power = 0x80000000u >> (31u - shift);
  uint32_t restored = truncated * power;
  uint32_t remainder = significand - restored;
  uint32_t half = power >> 1;
  int above_half = half < remainder;
  int at_half = half == remainder;
  int odd = (truncated % 2u) == 1u;
  int round_up = above_half || (at_half && odd);
  uint32_t subnormal_bits = truncated + (round_up ? 1u : 0u);
  uint32_t offset = n * 0x00800000u;
  uint32_t down_bits = y_bits - offset;
  uint32_t up_bits = y_bits + offset;
  uint32_t down_result = subnormal ? subnormal_bits : down_bits;
  return bitsf(negative ? down_result : up_bits);
}

/* numeric.hex:63-102 (fdlibm-derived F32 exp). */
float ox_exp(float x) {
  uint32_t bits = fbits(x);
  uint32_t magnitude = bits % 0x80000000u;
  int negative = 0x80000000u <= bits;
  int nan = 0x7F800000u < magnitude;
  uint32_t limit = negative ? 0x42CFF1B5u : 0x42B17218u;
  int finite_range = magnitude < limit;
  float safe_x = finite_range ? x : 0.0f;
  float absolute = negative ? -safe_x : safe_x;
  float scaled = absolute * bitsf(0x3FB8AA3Bu);
  uint32_t n = round_u32(scaled);
  float nf = (float)n;
  float k = negative ? -nf : nf;
  float k_hi = k * bitsf(0x3F317200u);
  float hi = safe_x - k_hi;
  float lo = k * bitsf(0x35BFBE8Eu);
  float r = hi - lo;
  float square = r * r;
  float p2_term = square * bitsf(0xBB355215u);
  float polynomial = bitsf(0x3E2AAA8Fu) + p2_term;
  float correction = square * polynomial;
  float c = r - correction;
  float numerator = r * c;
  float denominator = 2.0f - c;
  float ratio = numerator / denominator;
  float tail = lo - ratio;
  float adjustment = tail - hi;
  float y = 1.0f - adjustment;
  float scaled_result = exp_scale(y, n, negative);
  int tiny = magnitude < 0x39000000u;
  float tiny_result = 1.0f + safe_x;
  float finite_result = tiny ? tiny_result : scaled_result;
  float exceptional = negative ? 0.0f : bitsf(0x7F800000u);
  float classified = finite_range ? finite_result : exceptional;
  return nan ? bitsf(0x7FC00000u) : classified;
}

/* numeric.hex:104-113 */
float ox_silu(float x) { return x / (1.0f + ox_exp(-x)); }
/* numeric.hex:115-124 */
float ox_sigmoid(float x) { return 1.0f / (1.0f + ox_exp(-x)); }

/* numeric.hex:126-174: max(x,0) + 2*atanh(e/(2+e)), e = exp(-|x|). */
float ox_softplus(float x) {
  int positive = x > 0.0f;
  float maximum = positive ? x : 0.0f;
  float negative_absolute = positive ? -x : x;
  float e = ox_exp(negative_absolute);
  float z = e / (2.0f + e);
  float z2 = z * z;
  float p = bitsf(0x3D888889u) + z2 * bitsf(0x3D70F0F1u);
  p = bitsf(0x3D9D89D9u) + z2 * p;
  p = bitsf(0x3DBA2E8Cu) + z2 * p;
  p = bitsf(0x3DE38E39u) + z2 * p;
  p = bitsf(0x3E124925u) + z2 * p;
  p = bitsf(0x3E4CCCCDu) + z2 * p;
  p = bitsf(0x3EAAAAABu) + z2 * p;
  p = 1.0f + z2 * p;
  float half_log = z * p;
  float logarithm = 2.0f * half_log;
  return maximum + logarithm;
}

/* numeric.hex:176-206: exponent-halving guess, four Newton steps. */
float ox_sqrt(float x) {
  float g = bitsf((fbits(x) >> 1) + 0x1FC00000u);
  for (int i = 0; i < 4; ++i) g = (g + x / g) * 0.5f;
  return x <= 0.0f ? 0.0f : g;
}

/* numeric.hex:208-287: three-part pi/2 reduction, degree-13/14 polynomials. */
void ox_sincos(float angle, float* sine, float* cosine) {
  uint32_t q = round_u32(angle * bitsf(0x3F22F983u));
  float qf = (float)q;
  float r = angle - qf * bitsf(0x3FC90000u);
  r = r - qf * bitsf(0x39FDA000u);
  r = r - qf * bitsf(0x33A22169u);
  float s2 = r * r;
  float sp = bitsf(0xB2D72F34u) + s2 * bitsf(0x2F2EC9D3u);
  sp = bitsf(0x3638EF1Bu) + s2 * sp;
  sp = bitsf(0xB9500D01u) + s2 * sp;
  sp = bitsf(0x3C088889u) + s2 * sp;
  sp = bitsf(0xBE2AAAABu) + s2 * sp;
  float s = r + (r * s2) * sp;
  float cp = bitsf(0x310F74F6u) + s2 * bitsf(0xAD47D74Eu);
  cp = bitsf(0xB493F27Cu) + s2 * cp;
  cp = bitsf(0x37D00D01u) + s2 * cp;
  cp = bitsf(0xBAB60B61u) + s2 * cp;
  cp = bitsf(0x3D2AAAABu) + s2 * cp;
  float c = (1.0f - s2 * 0.5f) + (s2 * s2) * cp;
  switch (q % 4u) {
    case 0: *sine = s; *cosine = c; break;
    case 1: *sine = c; *cosine = -s; break;
    case 2: *sine = -s; *cosine = -c; break;
    default: *sine = -c; *cosine = s; break;
  }
}

/* ------------------------------------------------------------ reductions */

/* Halving tree over `width` lane values (cooperative.hex:275-335). */
static float tree(float* v, int width) {
  for (int stride = width >> 1; stride >= 1; stride >>= 1)
    for (int l = 0; l < stride; ++l) v[l] += v[l + stride];
  return v[0];
}

/* Split low/high accumulation, lane l visits pairs l, l+W, ... then a
 * halving tree of width W (tests/qwen35_simt.rs:99-116; the S32/S64/S256
 * trees of qwen35_simt.hex:4-120, 240-346). */
float ox_dot_width(const uint16_t* x, const uint16_t* w, int64_t pairs, int width) {
  float sums[256];
  for (int lane = 0; lane < width; ++lane) {
    float lo = 0.0f, hi = 0.0f;
    for (int64_t p = lane; p < pairs; p += width) {
      lo += ox_bf2f(x[2 * p]) * ox_bf2f(w[2 * p]);
      hi += ox_bf2f(x[2 * p + 1]) * ox_bf2f(w[2 * p + 1]);
    }
    sums[lane] = lo + hi;
  }
  return tree(sums, width);
}

/* Same tree with F32 weights: the MoE router (qwen35_simt.hex:122-239). */
float ox_dot_width_f32w(const uint16_t* x, const float* w, int64_t pairs, int width) {
  float sums[256];
  for (int lane = 0; lane < width; ++lane) {
    float lo = 0.0f, hi = 0.0f;
    for (int64_t p = lane; p < pairs; p += width) {
      lo += ox_bf2f(x[2 * p]) * w[2 * p];
      hi += ox_bf2f(x[2 * p + 1]) * w[2 * p + 1];
    }
    sums[lane] = lo + hi;
  }
  return tree(sums, width);
}

/* Dual split-pair dot sharing the input (simt.hex:301-346). */
static void dot_dual(const uint16_t* x, const uint16_t* w1, const uint16_t* w2, int64_t pairs,
                     int width, float* r1, float* r2) {
  float a[256], b[256];
  for (int lane = 0; lane < width; ++lane) {
    float l1 = 0.0f, h1 = 0.0f, l2 = 0.0f, h2 = 0.0f;
    for (int64_t p = lane; p < pairs; p += width) {
      float xl = ox_bf2f(x[2 * p]), xh = ox_bf2f(x[2 * p + 1]);
      l1 += xl * ox_bf2f(w1[2 * p]);
      h1 += xh * ox_bf2f(w1[2 * p + 1]);
      l2 += xl * ox_bf2f(w2[2 * p]);
      h2 += xh * ox_bf2f(w2[2 * p + 1]);
    }
    a[lane] = l1 + h1;
    b[lane] = l2 + h2;
  }
  *r1 = tree(a, width);
  *r2 = tree(b, width);
}

/* B256, the batched-prefill projections: lane l visits pairs l, l+256, ...
 * with ONE accumulator, acc = (acc + x.lo*w.lo) + x.hi*w.hi (bf16x2.dot-f32,
 * numeric.hex:17-28), then the 256-wide halving tree (batch_projection.hex:
 * 4-18 and 855-941; cooperative.hex:285-335). Lanes without pairs hold +0. */
float ox_dot_b256(const uint16_t* x, const uint16_t* w, int64_t pairs) {
  float sums[256];
  for (int lane = 0; lane < 256; ++lane) {
    float acc = 0.0f;
    for (int64_t p = lane; p < pairs; p += 256) {
      acc = acc + ox_bf2f(x[2 * p]) * ox_bf2f(w[2 * p]);
      acc = acc + ox_bf2f(x[2 * p + 1]) * ox_bf2f(w[2 * p + 1]);
    }
    sums[lane] = acc;
  }
  return tree(sums, 256);
}

/* Dual B256 sharing the input (batch.dot-dual, batch_projection.hex:4-18). */
static void dot_b256_dual(const uint16_t* x, const uint16_t* w1, const uint16_t* w2, int64_t pairs,
                          float* r1, float* r2) {
  float a[256], b[256];
  for (int lane = 0; lane < 256; ++lane) {
    float g = 0.0f, u = 0.0f;
    for (int64_t p = lane; p < pairs; p += 256) {
      float xl = ox_bf2f(x[2 * p]), xh = ox_bf2f(x[2 * p + 1]);
      g = g + xl * ox_bf2f(w1[2 * p]);
      g = g + xh * ox_bf2f(w1[2 * p + 1]);
      u = u + xl * ox_bf2f(w2[2 * p]);
      u = u + xh * ox_bf2f(w2[2 * p + 1]);
    }
    a[lane] = g;
    b[lane] = u;
  }
  *r1 = tree(a, 256);
  *r2 = tree(b, 256);
}

static int64_t next_pow2(int64_t v) { int64_t p = 1; while (p < v) p <<= 1; return p; }

/* Adjacent-pair tree of x^2 over the padded power-of-two width
 * (qwen35.hex:834-900; full_prepare.hex:20-31). */
static float ap_sum_squares(const uint16_t* x, int64_t cols) {
  int64_t pad = next_pow2(cols);
  float* buf = (float*)malloc(sizeof(float) * (size_t)pad);
  for (int64_t i = 0; i < pad; ++i) {
    float v = i < cols ? ox_bf2f(x[i]) : 0.0f;
    buf[i] = i < cols ? v * v : 0.0f;
  }
  for (int64_t d = 1; d < pad; d <<= 1)
    for (int64_t left = 0; left + d < pad; left += 2 * d) buf[left] += buf[left + d];
  float s = buf[0];
  free(buf);
  return s;
}

/* qwen35.normalize (qwen35.hex:912-977) with the write of
 * fused_normalization.hex:25-41: y = bf16(x*inv) (x) bf16(w). */
static void normalize_rows(const uint16_t* x, const float* w, int64_t cols, int64_t rows,
                           float eps, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * cols;
    float sum = ap_sum_squares(xr, cols);
    float mean = sum / (float)cols;
    float inverse = 1.0f / ox_sqrt(mean + eps);
    for (int64_t c = 0; c < cols; ++c)
      out[r * cols + c] = bf_mul(ox_f2bf(ox_bf2f(xr[c]) * inverse),
                                 ox_f2bf(g_plant == OX_PLANT_NORM_WEIGHT ? 1.0f : w[c]));
  }
}

/* ------------------------------------------------------- weight ABI */

enum {
  K_EMBED = 0, K_MATRIX, K_NORM, K_DT, K_A, K_CONV, K_ROUTER, K_SHARED_GATE
};

static int is_full(const ox_config* c, int l) { return ((l + 1) % c->full_interval) == 0; }
static int layer_count(const ox_config* c, int l) {
  return is_full(c, l) ? (c->moe ? 16 : 11) : (c->moe ? 19 : 14);
}

int64_t ox_weight_count(const ox_config* c) {
  int64_t n = 1;
  for (int l = 0; l < c->layers; ++l) n += layer_count(c, l);
  return n + 2;
}

/* src/spec.rs:443-712, in order. */
int ox_weight_info(const ox_config* c, int64_t index, int32_t* dtype, int64_t* rows,
                   int64_t* cols, int32_t* kind) {
  const int64_t H = c->hidden, HD = c->head_dim;
  const int64_t KS = (int64_t)c->key_heads * c->key_dim;
  const int64_t VS = (int64_t)c->value_heads * c->value_dim;
  const int64_t QKV = 2 * KS + VS;
  int64_t total = ox_weight_count(c);
  if (index < 0 || index >= total) return -1;
#define SET(d, r, co, k) do { *dtype = (d); *rows = (r); *cols = (co); *kind = (k); return 0; } while (0)
  if (index == 0) SET(OX_BF16, c->vocab, H, K_EMBED);
  if (index == total - 2) SET(OX_F32, H, 1, K_NORM);
  if (index == total - 1) SET(OX_BF16, c->vocab, H, K_EMBED);
  int64_t base = 1;
  for (int l = 0; l < c->layers; ++l) {
    int n = layer_count(c, l);
    if (index < base + n) {
      int s = (int)(index - base);
      if (s == 0) SET(OX_F32, H, 1, K_NORM);
      int ffn;
      if (is_full(c, l)) {
        switch (s) {
          case 1: SET(OX_BF16, 2 * (int64_t)c->q_heads * HD, H, K_MATRIX);
          case 2: SET(OX_BF16, (int64_t)c->kv_heads * HD, H, K_MATRIX);
          case 3: SET(OX_BF16, (int64_t)c->kv_heads * HD, H, K_MATRIX);
          case 4: SET(OX_BF16, H, (int64_t)c->q_heads * HD, K_MATRIX);
          case 5: SET(OX_F32, HD, 1, K_NORM);
          case 6: SET(OX_F32, HD, 1, K_NORM);
          case 7: SET(OX_F32, H, 1, K_NORM);
        }
        ffn = s - 8;
      } else {
        switch (s) {
          case 1: SET(OX_BF16, QKV, H, K_MATRIX);
          case 2: SET(OX_BF16, VS, H, K_MATRIX);
          case 3: SET(OX_BF16, c->value_heads, H, K_MATRIX);
          case 4: SET(OX_BF16, c->value_heads, H, K_MATRIX);
          case 5: SET(OX_F32, c->value_heads, 1, K_DT);
          case 6: SET(OX_F32, c->value_heads, 1, K_A);
          case 7: SET(OX_F32, c->value_dim, 1, K_NORM);
          case 8: SET(OX_BF16, H, VS, K_MATRIX);
          case 9: SET(OX_F32, QKV, 4, K_CONV);
          case 10: SET(OX_F32, H, 1, K_NORM);
        }
        ffn = s - 11;
      }
      const int64_t I = c->intermediate, E = c->experts, SI = c->shared_intermediate;
      if (!c->moe) {
        switch (ffn) {
          case 0: SET(OX_BF16, I, H, K_MATRIX);
          case 1: SET(OX_BF16, I, H, K_MATRIX);
          case 2: SET(OX_BF16, H, I, K_MATRIX);
        }
      } else {
        switch (ffn) {
          case 0: SET(OX_F32, E, H, K_ROUTER);
          case 1: SET(OX_BF16, E * I, H, K_MATRIX);
          case 2: SET(OX_BF16, E * I, H, K_MATRIX);
          case 3: SET(OX_BF16, E * H, I, K_MATRIX);
          case 4: SET(OX_F32, 1, H, K_SHARED_GATE);
          case 5: SET(OX_BF16, SI, H, K_MATRIX);
          case 6: SET(OX_BF16, SI, H, K_MATRIX);
          case 7: SET(OX_BF16, H, SI, K_MATRIX);
        }
      }
      return -1;
    }
    base += n;
  }
#undef SET
  return -1;
}

/* ------------------------------------------------- synthetic weights */

/* Synthetic-weight specification (the GPU library implements the same
 * formulas independently): a SplitMix64 finaliser keyed by (seed, tensor)
 * and counted by element; an approximately normal variate is the centred sum
 * of the four 16-bit fields (Irwin-Hall, n=4), scaled by one F32 multiply. */
uint64_t ox_mix64(uint64_t x) {
  x ^= x >> 30; x *= 0xBF58476D1CE4E5B9ull;
  x ^= x >> 27; x *= 0x94D049BB133111EBull;
  x ^= x >> 31;
  return x;
}
static inline uint64_t elem_hash(uint64_t key, uint64_t i) {
  return ox_mix64(key + i * 0x9E3779B97F4A7C15ull);
}
static inline int32_t centred(uint64_t h) {
  int32_t s = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) +
              (int32_t)((h >> 32) & 0xFFFF) + (int32_t)(h >> 48);
  return s - 131070;
}
static float normal_scale(double sd) { return (float)(sd / sqrt(1431655765.0)); }

void ox_fill_tensor(const ox_config* c, uint64_t seed, int64_t index, void* dst) {
  int32_t dtype, kind;
  int64_t rows, cols;
  if (ox_weight_info(c, index, &dtype, &rows, &cols, &kind) != 0) return;
  int64_t source = index;
  if (c->tied && index == ox_weight_count(c) - 1) source = 0;  /* lm_head = token_embd */
  uint64_t key = ox_mix64(seed ^ ox_mix64((uint64_t)source + 1));
  int64_t count = rows * cols;
  float s02 = normal_scale(0.02), s_conv = normal_scale(0.3), s_router = normal_scale(0.04);
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < count; ++i) {
    uint64_t h = elem_hash(key, (uint64_t)i);
    switch (kind) {
      case K_EMBED:
      case K_MATRIX:
        ((uint16_t*)dst)[i] = ox_f2bf((float)centred(h) * s02);
        break;
      case K_NORM: ((float*)dst)[i] = 1.0f + (float)centred(h) * s02; break;
      case K_DT: ((float*)dst)[i] = 1.0f; break;
      case K_A: {
        float u = (float)(uint32_t)(h >> 40) * 0x1p-24f;
        ((float*)dst)[i] = -(1.0f + 15.0f * u);
        break;
      }
      case K_CONV: ((float*)dst)[i] = (float)centred(h) * s_conv; break;
      case K_ROUTER: ((float*)dst)[i] = (float)centred(h) * s_router; break;
      default: ((float*)dst)[i] = (float)centred(h) * s02; break;
    }
  }
}

/* ------------------------------------------------------------- model */

struct ox_model {
  ox_config c;
  void* const* w;
  int64_t KS, VS, QKV, REC, CONV, LIN, KVS, QS;
  float* freq;           /* F32 theta^(-2i/R), src/catena.rs:185-232 */
  int64_t* layer_base;   /* first weight index of each layer */
};

ox_model* ox_model_create(const ox_config* c, void* const* weights) {
  ox_model* m = (ox_model*)calloc(1, sizeof(ox_model));
  m->c = *c;
  m->w = weights;
  m->KS = (int64_t)c->key_heads * c->key_dim;
  m->VS = (int64_t)c->value_heads * c->value_dim;
  m->QKV = 2 * m->KS + m->VS;
  m->REC = m->VS * c->key_dim;
  m->CONV = 3 * m->QKV;
  m->LIN = m->CONV + m->REC;
  m->KVS = (int64_t)c->kv_heads * c->head_dim;
  m->QS = (int64_t)c->q_heads * c->head_dim;
  int half = c->rope_dim / 2;
  m->freq = (float*)malloc(sizeof(float) * (size_t)(half > 0 ? half : 1));
  for (int i = 0; i < half; ++i)
    m->freq[i] = powf(c->theta, -((float)(2 * i) / (float)c->rope_dim));
  m->layer_base = (int64_t*)malloc(sizeof(int64_t) * (size_t)c->layers);
  int64_t b = 1;
  for (int l = 0; l < c->layers; ++l) { m->layer_base[l] = b; b += layer_count(c, l); }
  return m;
}

void ox_model_free(ox_model* m) {
  if (!m) return;
  free(m->freq);
  free(m->layer_base);
  free(m);
}

static const void* W(const ox_model* m, int l, int slot) { return m->w[m->layer_base[l] + slot]; }
#define WB(m, l, s) ((const uint16_t*)W(m, l, s))
#define WF(m, l, s) ((const float*)W(m, l, s))

int64_t ox_cache_elements(const ox_config* c, int64_t capacity) {
  /* src/spec.rs:321-362 (= state_layout.hex:26-27). */
  int64_t KS = (int64_t)c->key_heads * c->key_dim;
  int64_t VS = (int64_t)c->value_heads * c->value_dim;
  int64_t QKV = 2 * KS + VS;
  int64_t kv = capacity * (int64_t)c->layers * 2 * c->kv_heads * c->head_dim;
  return kv + (int64_t)c->layers * (3 * QKV + VS * c->key_dim);
}

struct ox_session {
  const ox_model* m;
  int64_t capacity;
  uint16_t* cache;
  float* shadow;
  int64_t* last_ids;
  int64_t split_keys;  /* decode attention over more keys than this splits (0: never) */
};

ox_session* ox_session_create(const ox_model* m, int64_t capacity) {
  ox_session* s = (ox_session*)calloc(1, sizeof(ox_session));
  s->m = m;
  s->capacity = capacity;
  s->cache = (uint16_t*)calloc((size_t)ox_cache_elements(&m->c, capacity), 2);
  s->shadow = (float*)calloc((size_t)(m->REC * m->c.layers), 4);
  s->last_ids = (int64_t*)calloc((size_t)(m->c.layers * (m->c.top_k > 0 ? m->c.top_k : 1)), 8);
  s->split_keys = OX_SPLIT_KEYS_DEFAULT;
  return s;
}
void ox_session_set_split_keys(ox_session* s, int64_t keys) { s->split_keys = keys; }
void ox_session_free(ox_session* s) {
  if (!s) return;
  free(s->cache); free(s->shadow); free(s->last_ids); free(s);
}
uint16_t* ox_session_cache(ox_session* s) { return s->cache; }
float* ox_session_shadow(ox_session* s) { return s->shadow; }
const int64_t* ox_session_last_ids(const ox_session* s) { return s->last_ids; }

/* GEMV over a row-major BF16 matrix, each row a split-pair tree of `width`. */
static void gemv(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols, int width,
                 float* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) out[r] = ox_dot_width(x, w + r * cols, cols / 2, width);
}

/* qwen3.fused.project / group-project: bf16(tree) (simt.hex:400-410). */
static void project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols, int width,
                    uint16_t* out) {
  float* t = (float*)malloc(sizeof(float) * (size_t)rows);
  gemv(x, w, rows, cols, width, t);
  for (int64_t r = 0; r < rows; ++r) out[r] = ox_f2bf(t[r]);
  free(t);
}

/* qwen3.fused.residual: bf16(bf16(tree64) (+) residual) (simt.hex:442-538). */
static void residual_project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols,
                             const uint16_t* residual, uint16_t* out) {
  float* t = (float*)malloc(sizeof(float) * (size_t)rows);
  gemv(x, w, rows, cols, 64, t);
  for (int64_t r = 0; r < rows; ++r) out[r] = bf_add(ox_f2bf(t[r]), residual[r]);
  free(t);
}

/* qwen3.fused.gate: bf16(silu(bf16 g)) (x) bf16(u), S256 dual (simt.hex:539-646). */
static void swiglu_project(const uint16_t* x, const uint16_t* wg, const uint16_t* wu, int64_t rows,
                           int64_t cols, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    float g, u;
    dot_dual(x, wg + r * cols, wu + r * cols, cols / 2, 256, &g, &u);
    uint16_t a = ox_f2bf(ox_silu(rbf(g)));
    out[r] = bf_mul(a, ox_f2bf(u));
  }
}

/* qwen3.rope-one (rope.hex:5-17, 43-55): [cos x R/2 | sin x R/2]. */
static void rope_table(const ox_model* m, int64_t position, float* table) {
  int half = m->c.rope_dim / 2;
  float p = (float)(uint32_t)position;
  for (int i = 0; i < half; ++i) {
    float s, c;
    float f = m->freq[i];
    if (g_plant == OX_PLANT_ROPE_FREQ_HD) f = powf(m->c.theta, -((float)(2 * i) / (float)m->c.head_dim));
    ox_sincos(p * f, &s, &c);
    table[i] = c;
    table[half + i] = s;
  }
}

/* neox rotation of one head (rope.hex:56-82; full_prepare.hex:49-63). */
static void rotate_head(const uint16_t* in, const float* table, int HD, int R, uint16_t* out) {
  int half = R / 2;
  for (int c = 0; c < HD; ++c) {
    float a = ox_bf2f(in[c]);
    float v = a;
    if (c < R) {
      int pair = c % half;
      int first = c < half;
      float b = ox_bf2f(in[first ? pair + half : pair]);
      if (g_plant == OX_PLANT_ROPE_PAIRING) {  /* interleaved (2i, 2i+1) pairs */
        pair = c / 2;
        first = (c & 1) == 0;
        b = ox_bf2f(in[first ? c + 1 : c - 1]);
      }
      float ac = a * table[pair];
      float bs = b * table[pair + half];
      v = first ? ac - bs : ac + bs;
      if (g_plant == OX_PLANT_ROPE_SIGN) v = first ? ac + bs : ac - bs;
    }
    out[c] = ox_f2bf(v);
  }
}

typedef struct {
  uint16_t *h, *x, *attn;                 /* H */
  uint16_t *qkv, *conv, *z, *alpha, *beta; /* linear */
  uint16_t *q, *k, *core, *gated;
  uint16_t *qg, *kraw, *vraw, *qn, *kn, *qr, *kr, *ctx; /* full */
  float *scores, *f32tmp, *rope;
  uint16_t *probs16;
  uint16_t *active;
  float *router;
} scratch_t;

/* 4-tap causal conv + history (qwen35.hex:278-340; linear_prepare.hex:2-64). */
static void conv_step(const ox_model* m, uint16_t* cache, int64_t conv_base, int64_t position,
                      const float* weight, const uint16_t* qkv, uint16_t* out) {
  const int64_t QKV = m->QKV;
  for (int64_t ch = 0; ch < QKV; ++ch) {
    float taps[3];
    for (int t = 0; t < 3; ++t) {
      int64_t p = position + t;
      float hist = ox_bf2f(cache[conv_base + (p % 3) * QKV + ch]);
      float input = p < 3 ? 0.0f : hist;
      taps[t] = input * weight[ch * 4 + (g_plant == OX_PLANT_CONV_TAP_ORDER ? 3 - t : t)];
    }
    float tap3 = ox_bf2f(qkv[ch]) * weight[ch * 4 + (g_plant == OX_PLANT_CONV_TAP_ORDER ? 0 : 3)];
    float sum = (taps[0] + taps[2]) + (taps[1] + tap3);
    out[ch] = ox_f2bf(ox_silu(rbf(sum)));
  }
  for (int64_t ch = 0; ch < QKV; ++ch) cache[conv_base + (position % 3) * QKV + ch] = qkv[ch];
}

/* Per-head L2 norm with a serial sum (qwen35.hex:396-436; linear_prepare.hex:84-131). */
static void l2_heads(const uint16_t* in, int heads, int dim, uint16_t* out) {
  if (g_plant == OX_PLANT_L2_WHOLE) { dim *= heads; heads = 1; }
  for (int h = 0; h < heads; ++h) {
    float sum = 0.0f;
    for (int i = 0; i < dim; ++i) { float v = ox_bf2f(in[h * dim + i]); sum += v * v; }
    float norm = ox_sqrt(sum + bitsf(0x358637BDu));
    for (int i = 0; i < dim; ++i) out[h * dim + i] = ox_f2bf(ox_bf2f(in[h * dim + i]) / norm);
  }
}

/* Gated DeltaNet single step for every value channel (cached_delta.hex:69-135,
 * register_delta.hex:5-124, fused_delta.hex:1-20). State rows are BF16 in the
 * cache (decode) or F32 in the shadow (multi-token call). */
static void delta_step(const ox_model* m, const uint16_t* conv, const uint16_t* q, const uint16_t* k,
                       const uint16_t* alpha, const uint16_t* beta, const float* dt, const float* a,
                       uint16_t* state16, float* state32, uint16_t* out) {
  const int KD = m->c.key_dim, VD = m->c.value_dim, KH = m->c.key_heads;
  const int64_t VS = m->VS, KS = m->KS;
  const float scale = g_plant == OX_PLANT_DELTA_SCALE ? 1.0f : 1.0f / sqrtf((float)KD);  /* DELTA_SCALE_BITS, qwen35.rs:703 */
  const int ratio = m->c.value_heads / KH;
#pragma omp parallel for schedule(static)
  for (int64_t c = 0; c < VS; ++c) {
    int head = (int)(c / VD);
    int kbase = (g_plant == OX_PLANT_KEY_HEAD ? head / ratio : head % KH) * KD;
    float time_step = ox_softplus(ox_bf2f(alpha[head]) + dt[head]);
    float decay = ox_exp(rbf(time_step * a[head]));
    float rate = rbf(ox_sigmoid(ox_bf2f(beta[head])));
    float lanes[32];
    float old[1024];
    for (int i = 0; i < KD; ++i)
      old[i] = state16 ? ox_bf2f(state16[c * KD + i]) : state32[c * KD + i];
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int i = l; i < KD; i += 32) acc += old[i] * ox_bf2f(k[kbase + i]);
      lanes[l] = acc;
    }
    float total = tree(lanes, 32);
    float value = ox_bf2f(conv[2 * KS + c]);
    float delta = (value - (g_plant == OX_PLANT_DELTA_PRED_DECAY ? total : total * decay)) * rate;
    for (int l = 0; l < 32; ++l) {
      float acc = 0.0f;
      for (int i = l; i < KD; i += 32) {
        float next = old[i] * decay + ox_bf2f(k[kbase + i]) * delta;
        if (state16) state16[c * KD + i] = ox_f2bf(next);
        else state32[c * KD + i] = next;
        acc += next * ox_bf2f(q[kbase + i]);
      }
      lanes[l] = acc;
    }
    out[c] = ox_f2bf(tree(lanes, 32) * scale);
  }
}

/* Gated RMSNorm x SiLU(z), serial sum per head (qwen35.hex:753-778;
 * cooperative_norm.hex:139-182). */
static void gated_norm(const ox_model* m, const uint16_t* core, const uint16_t* z, const float* w,
                       uint16_t* out) {
  const int VD = m->c.value_dim;
  for (int h = 0; h < m->c.value_heads; ++h) {
    float sum = 0.0f;
    for (int i = 0; i < VD; ++i) { float v = ox_bf2f(core[h * VD + i]); sum += v * v; }
    float rms = ox_sqrt((g_plant == OX_PLANT_GATED_SUM ? sum : sum / (float)VD) + m->c.eps);
    for (int i = 0; i < VD; ++i) {
      float normalized = ox_bf2f(core[h * VD + i]) / rms;
      float gate = ox_silu(ox_bf2f(z[h * VD + i]));
      out[h * VD + i] = ox_f2bf((normalized * w[i]) * gate);
    }
  }
}

/* Online decode attention, 8-key tiles (online.hex:4-331).
 *
 * Split-K above split_keys keys (this build's long-context mode; the
 * reference always runs one chain): the T tiles form at most 128 ranges of
 * ceil(T / 128) tiles each (the last may be shorter), and each range runs
 * the reference's online recurrence over its own tiles
 * from scratch (running maximum m_r, den_r = den_r a + p_0 + ... + p_7,
 * acc_r = acc_r a + p_0 v_0 + ...). The ranges merge in ascending order:
 * M = max_r m_r, w_r = exp(m_r - M), den = (0 + den_0 w_0) + den_1 w_1 + ...,
 * acc likewise; out = bf16(bf16(acc / den) * sigmoid(gate)). At or below
 * split_keys (and with split_keys = 0) the single chain is the reference's. */
#define OX_SPLIT_RANGES 128
static void attention_online(const ox_model* m, const uint16_t* q, const uint16_t* cache,
                             int64_t key_base, int64_t value_base, int64_t keys,
                             const uint16_t* qg, int64_t split_keys, uint16_t* out) {
  const int HD = m->c.head_dim, hpk = m->c.q_heads / m->c.kv_heads;
  const int64_t KVS = m->KVS;
  const int split = split_keys > 0 && keys > split_keys;
  const int64_t tiles = (keys + 7) / 8;
  const int64_t range_tiles = split ? (tiles + OX_SPLIT_RANGES - 1) / OX_SPLIT_RANGES : tiles;
  const float scale = g_plant == OX_PLANT_ATTN_SCALE ? 1.0f : 1.0f / sqrtf((float)HD);  /* SCALE_BITS, qwen35.rs:701 */
#pragma omp parallel for schedule(static)
  for (int head = 0; head < m->c.q_heads; ++head) {
    int64_t off = (int64_t)(g_plant == OX_PLANT_GQA_MAP ? head % m->c.kv_heads : head / hpk) * HD;
    const int64_t nranges = (tiles + range_tiles - 1) / range_tiles;
    float* rmax = (float*)malloc(sizeof(float) * (size_t)nranges);
    float* rden = (float*)malloc(sizeof(float) * (size_t)nranges);
    float* racc = (float*)malloc(sizeof(float) * (size_t)(nranges * HD));
    for (int64_t r = 0; r < nranges; ++r) {
      float maximum = bitsf(0xFF800000u), den = 0.0f;
      float* acc = racc + r * HD;
      for (int ch = 0; ch < HD; ++ch) acc[ch] = 0.0f;
      const int64_t t_end = (r + 1) * range_tiles < tiles ? (r + 1) * range_tiles : tiles;
      for (int64_t t = r * range_tiles; t < t_end; ++t) {
        const int64_t first = t * 8;
        float score[8], p[8];
        for (int j = 0; j < 8; ++j) {
          int64_t key = first + j;
          if (key >= keys) { score[j] = bitsf(0xFF800000u); continue; }
          float lanes[32];
          for (int l = 0; l < 32; ++l) {
            float a = 0.0f;
            for (int ch = l; ch < HD; ch += 32)
              a += ox_bf2f(q[head * HD + ch]) * ox_bf2f(cache[key_base + key * KVS + off + ch]);
            lanes[l] = a;
          }
          score[j] = tree(lanes, 32) * scale;
        }
        float next_max = maximum;
        for (int j = 0; j < 8; ++j) next_max = fmaxf(next_max, score[j]);
        float alpha = ox_exp(maximum - next_max);
        den = den * alpha;
        for (int j = 0; j < 8; ++j) { p[j] = ox_exp(score[j] - next_max); den = den + p[j]; }
        maximum = next_max;
        for (int ch = 0; ch < HD; ++ch) {
          float v = acc[ch] * alpha;
          for (int j = 0; j < 8; ++j) {
            int64_t key = first + j < keys ? first + j : 0;
            v = v + p[j] * ox_bf2f(cache[value_base + key * KVS + off + ch]);
          }
          acc[ch] = v;
        }
      }
      rmax[r] = maximum;
      rden[r] = den;
    }
    float total = rden[0];
    float* value = racc;  /* one range: the reference's single chain */
    float* merged = NULL;
    if (split) {
      float M = bitsf(0xFF800000u);
      for (int64_t r = 0; r < nranges; ++r) M = fmaxf(M, rmax[r]);
      merged = (float*)calloc((size_t)HD, sizeof(float));
      total = 0.0f;
      for (int64_t r = 0; r < nranges; ++r) {
        const float w = ox_exp(rmax[r] - M);
        total = total + rden[r] * w;
        for (int ch = 0; ch < HD; ++ch) merged[ch] = merged[ch] + racc[r * HD + ch] * w;
      }
      value = merged;
    }
    for (int ch = 0; ch < HD; ++ch) {
      float gate = ox_sigmoid(ox_bf2f(qg[2 * (int64_t)head * HD + HD + ch]));
      out[head * HD + ch] = ox_f2bf(rbf(value[ch] / total) * gate);
    }
    free(rmax); free(rden); free(racc); free(merged);
  }
}

/* Staged dense attention: scalar-order scores (qwen35.rs:722-790,
 * attention.hex:71-92), softmax (qwen35_attention.hex:258-393), 8-way
 * interleaved context (qwen35_attention.hex:2-177), gate (qwen35.hex:207-222). */
static void attention_staged(const ox_model* m, const uint16_t* q, const uint16_t* cache,
                             int64_t key_base, int64_t value_base, int64_t keys,
                             const uint16_t* qg, uint16_t* out) {
  const int HD = m->c.head_dim, hpk = m->c.q_heads / m->c.kv_heads;
  const int64_t KVS = m->KVS;
  const float scale = g_plant == OX_PLANT_ATTN_SCALE ? 1.0f : 1.0f / sqrtf((float)HD);  /* ATTENTION_SCALE_BITS, mod.rs:361 */
  float* s = (float*)malloc(sizeof(float) * (size_t)keys);
  uint16_t* p = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)keys);
  float* buf = (float*)malloc(sizeof(float) * (size_t)keys);
  for (int head = 0; head < m->c.q_heads; ++head) {
    int64_t off = (int64_t)(g_plant == OX_PLANT_GQA_MAP ? head % m->c.kv_heads : head / hpk) * HD;
    for (int64_t key = 0; key < keys; ++key) {
      float acc = 0.0f;
      for (int i = 0; i < HD; ++i)
        acc += ox_bf2f(q[head * HD + i]) * ox_bf2f(cache[key_base + key * KVS + off + i]);
      s[key] = rbf(acc * scale);
    }
    float partial[256];
    for (int t = 0; t < 256; ++t) {
      float mx = bitsf(0xFF800000u);
      for (int64_t col = t; col < keys; col += 256) mx = fmaxf(mx, s[col]);
      partial[t] = mx;
    }
    for (int stride = 128; stride >= 1; stride >>= 1)
      for (int t = 0; t < stride; ++t) partial[t] = fmaxf(partial[t], partial[t + stride]);
    float maximum = partial[0];
    for (int64_t col = 0; col < keys; ++col) buf[col] = ox_exp(s[col] - maximum);
    for (int64_t d = 1; d < keys; d <<= 1)
      for (int64_t left = 0; left + d < keys; left += 2 * d) buf[left] += buf[left + d];
    float den = buf[0];
    for (int64_t col = 0; col < keys; ++col) p[col] = ox_f2bf(ox_exp(s[col] - maximum) / den);
    for (int ch = 0; ch < HD; ++ch) {
      float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      for (int64_t start = 0; start < keys; start += 8)
        for (int r = 0; r < 8; ++r) {
          int64_t key = start + r;
          if (key < keys)
            acc[r] = acc[r] + ox_bf2f(p[key]) * ox_bf2f(cache[value_base + key * KVS + off + ch]);
          else
            acc[r] = acc[r] + 0.0f;
        }
      float sum = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
      uint16_t context = ox_f2bf(sum);
      float gate = ox_sigmoid(ox_bf2f(qg[2 * (int64_t)head * HD + HD + ch]));
      out[head * HD + ch] = ox_f2bf(ox_bf2f(context) * gate);
    }
  }
  free(s); free(p); free(buf);
}

/* Router logits (E routed rows + the shared-expert gate row, S32 over BF16
 * input x F32 weights, moe.hex:4-84; the batched router runs the same stage
 * per token, batch_moe.hex:45-96) and the top-k selection: stable rank,
 * softmax over the selected logits with a serial denominator
 * (moe.hex:86-252; batch_moe.hex:136-281). */
/* Top-k of E router logits (moe.hex:86-252): expert e's rank is the number
 * of experts with a larger logit plus those with an equal logit and a lower
 * index (stable, ties toward the lower index); ids[rank] = e for rank < K;
 * p_j = exp(l_j - l_top) / den with den summed serially in rank order. NaN
 * logits can make two experts share a rank and leave another unassigned; an
 * unassigned rank k keeps expert k. */
static void select_top_k(const float* logit, int64_t E, int64_t K, int64_t* ids, float* prob) {
  float sel[64];
  for (int64_t j = 0; j < K; ++j) { ids[j] = j; sel[j] = logit[j]; }
  for (int64_t e = 0; e < E; ++e) {
    int64_t rank = 0;
    for (int64_t i = 0; i < E; ++i) {
      int larger = logit[i] > logit[e];
      int smaller = logit[e] > logit[i];
      if (g_plant == OX_PLANT_SELECT_ASCENDING) { int t = larger; larger = smaller; smaller = t; }
      int before = g_plant == OX_PLANT_SELECT_TIE_HIGH ? i > e : i < e;
      rank += larger ? 1 : ((before && !smaller) ? 1 : 0);
    }
    if (rank < K) { ids[rank] = e; sel[rank] = logit[e]; }
  }
  float ex[64], den = 0.0f;
  for (int64_t j = 0; j < K; ++j) ex[j] = ox_exp(sel[j] - sel[0]);
  if (g_plant == OX_PLANT_SOFTMAX_ALL)
    for (int64_t e = 0; e < E; ++e) den = den + ox_exp(logit[e] - sel[0]);
  else
    for (int64_t j = 0; j < K; ++j) den = den + ex[j];
  for (int64_t j = 0; j < K; ++j) prob[j] = g_plant == OX_PLANT_PROB_UNNORMALISED ? ex[j] : ex[j] / den;
}

static void moe_route(const ox_model* m, const uint16_t* x, const float* router,
                      const float* shared_router, int64_t* ids, float* prob, float* shared_prob) {
  const int64_t H = m->c.hidden, E = m->c.experts, K = m->c.top_k;
  float* logit = (float*)malloc(sizeof(float) * (size_t)(E + 1));
#pragma omp parallel for schedule(static)
  for (int64_t e = 0; e <= E; ++e)
    logit[e] = ox_dot_width_f32w(x, e < E ? router + e * H : shared_router, H / 2, 32);
  select_top_k(logit, E, K, ids, prob);
  *shared_prob = g_plant == OX_PLANT_SHARED_GATE ? 1.0f : ox_sigmoid(logit[E]);
  free(logit);
}

/* Expert gate/up rows: routed bf16(silu(g)*u*p), shared
 * bf16(bf16(bf16(silu(g))*u)*sigmoid) with g, u = bf16 of the dual dot:
 * S256 split pair in decode (moe.hex:254-333), B256 single accumulator in
 * the batched prefill (batch_moe.hex:339-411). */
static void moe_gate(const ox_model* m, int l, int ffn, const uint16_t* x, const int64_t* ids,
                     const float* prob, float shared_prob, int b256, uint16_t* active) {
  const int64_t H = m->c.hidden, K = m->c.top_k, I = m->c.intermediate,
                SI = m->c.shared_intermediate;
  const uint16_t* gate = WB(m, l, ffn + 1);
  const uint16_t* up = WB(m, l, ffn + 2);
  const uint16_t* sgate = WB(m, l, ffn + 5);
  const uint16_t* sup = WB(m, l, ffn + 6);
  const int64_t rows = K * I + SI;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    int routed = r < K * I;
    const uint16_t *wg, *wu;
    int64_t slot = 0;
    if (routed) {
      slot = r / I;
      int64_t row = ids[slot] * I + r % I;
      wg = gate + row * H; wu = up + row * H;
    } else {
      wg = sgate + (r - K * I) * H; wu = sup + (r - K * I) * H;
    }
    float g, u;
    if (b256) dot_b256_dual(x, wg, wu, H / 2, &g, &u);
    else dot_dual(x, wg, wu, H / 2, 256, &g, &u);
    float gb = rbf(g), ub = rbf(u);
    float activated = ox_silu(gb);
    float y;
    if (routed) y = (activated * ub) * prob[slot];
    else y = rbf(rbf(activated) * ub) * shared_prob;
    active[r] = ox_f2bf(y);
  }
}

/* Expert down: routed tree over the concatenated expert rows, shared tree,
 * then bf16(bf16(routed + residual) (+) bf16(shared)). Decode: S32 split
 * pair (moe.hex:371-434, simt_moe.hex:36-287); batched prefill: B256 single
 * accumulators, the shared terms gated to p < SI/2 inside the routed loop
 * (batch_moe.hex:453-563). */
static void moe_down(const ox_model* m, int l, int ffn, const uint16_t* active, const int64_t* ids,
                     const uint16_t* residual, int b256, uint16_t* out) {
  const int64_t H = m->c.hidden, K = m->c.top_k, I = m->c.intermediate,
                SI = m->c.shared_intermediate;
  const uint16_t* down = WB(m, l, ffn + 3);
  const uint16_t* sdown = WB(m, l, ffn + 7);
  const int64_t ip = I / 2, ap = K * I / 2, sp = SI / 2;
#pragma omp parallel for schedule(static)
  for (int64_t o = 0; o < H; ++o) {
    float routed, shared;
    if (b256) {
      float rl[256], sl[256];
      for (int lane = 0; lane < 256; ++lane) {
        float r = 0.0f, sh = 0.0f;
        for (int64_t p = lane; p < ap; p += 256) {
          const uint16_t* w = down + (ids[p / ip] * H + o) * I + 2 * (p % ip);
          r = r + ox_bf2f(active[2 * p]) * ox_bf2f(w[0]);
          r = r + ox_bf2f(active[2 * p + 1]) * ox_bf2f(w[1]);
          if (p < sp) {
            const uint16_t* sw = sdown + o * SI + 2 * p;
            const uint16_t* sx = active + K * I + 2 * p;
            sh = sh + ox_bf2f(sx[0]) * ox_bf2f(sw[0]);
            sh = sh + ox_bf2f(sx[1]) * ox_bf2f(sw[1]);
          }
        }
        rl[lane] = r;
        sl[lane] = sh;
      }
      routed = tree(rl, 256);
      shared = tree(sl, 256);
    } else {
      float lanes[32];
      for (int lane = 0; lane < 32; ++lane) {
        float lo = 0.0f, hi = 0.0f;
        for (int64_t p = lane; p < ap; p += 32) {
          const uint16_t* w = down + (ids[p / ip] * H + o) * I + 2 * (p % ip);
          lo += ox_bf2f(active[2 * p]) * ox_bf2f(w[0]);
          hi += ox_bf2f(active[2 * p + 1]) * ox_bf2f(w[1]);
        }
        lanes[lane] = lo + hi;
      }
      routed = tree(lanes, 32);
      shared = ox_dot_width(active + K * I, sdown + o * SI, sp, 32);
    }
    uint16_t routed_bf = ox_f2bf(routed + ox_bf2f(residual[o]));
    out[o] = bf_add(routed_bf, ox_f2bf(shared));
  }
}

/* Routed MoE FFN of one token (qwen35_moe.hex; graph qwen35.rs:124-167). */
static void moe_ffn(const ox_model* m, ox_session* se, int l, int ffn, const uint16_t* x,
                    const uint16_t* residual, int b256, uint16_t* out) {
  const int64_t K = m->c.top_k, I = m->c.intermediate, SI = m->c.shared_intermediate;
  int64_t ids[64];
  float prob[64], shared_prob;
  moe_route(m, x, WF(m, l, ffn + 0), WF(m, l, ffn + 4), ids, prob, &shared_prob);
  for (int64_t j = 0; j < K; ++j) se->last_ids[l * K + j] = ids[j];
  uint16_t* active = (uint16_t*)malloc(sizeof(uint16_t) * (size_t)(K * I + SI));
  moe_gate(m, l, ffn, x, ids, prob, shared_prob, b256, active);
  moe_down(m, l, ffn, active, ids, residual, b256, out);
  free(active);
}

static int argmax_bf16(const uint16_t* logits, int64_t vocab, uint64_t* token) {
  /* fused_argmax.hex: strict > from (0, -inf) over 256 contiguous chunks,
   * then a strict > reduce; the result is the first index of the maximum. */
  const int last = g_plant == OX_PLANT_ARGMAX_LAST;
  int64_t chunk = (vocab + 255) / 256;
  uint64_t best_tok = 0;
  float best = bitsf(0xFF800000u);
  for (int part = 0; part < 256; ++part) {
    int64_t base = (int64_t)part * chunk;
    uint64_t t = 0;
    float mx = bitsf(0xFF800000u);
    for (int64_t i = base; i < base + chunk && i < vocab; ++i) {
      float v = ox_bf2f(logits[i]);
      if (v > mx || (last && v == mx)) { mx = v; t = (uint64_t)i; }
    }
    if (mx > best || (last && mx == best && base < vocab)) { best = mx; best_tok = t; }
  }
  *token = best_tok;
  return 0;
}

static int64_t attention_interval_ok(const ox_config* c) { return c->full_interval > 0; }

/* ------------------------------------------------- batched prefill (K8) */

/* Token-major batched projections (batch.project / residual / gate,
 * batch_projection.hex:30-279, 280-530, 531-854): row r of token t is a B256
 * dot; epilogues bf16(total), bf16(bf16(total) (+) res), and
 * bf16(bf16(silu(bf16 g))) (x) bf16(u). */
static void bproject(const uint16_t* x, int64_t n, const uint16_t* w, int64_t rows, int64_t cols,
                     uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n * rows; ++i) {
    const int64_t t = i / rows, r = i % rows;
    out[i] = ox_f2bf(ox_dot_b256(x + t * cols, w + r * cols, cols / 2));
  }
}
static void bresidual(const uint16_t* x, int64_t n, const uint16_t* w, int64_t rows, int64_t cols,
                      const uint16_t* res, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n * rows; ++i) {
    const int64_t t = i / rows, r = i % rows;
    out[i] = bf_add(ox_f2bf(ox_dot_b256(x + t * cols, w + r * cols, cols / 2)), res[i]);
  }
}
static void bgate(const uint16_t* x, int64_t n, const uint16_t* wg, const uint16_t* wu,
                  int64_t rows, int64_t cols, uint16_t* out) {
#pragma omp parallel for schedule(static)
  for (int64_t i = 0; i < n * rows; ++i) {
    const int64_t t = i / rows, r = i % rows;
    float g, u;
    dot_b256_dual(x + t * cols, wg + r * cols, wu + r * cols, cols / 2, &g, &u);
    out[i] = bf_mul(ox_f2bf(ox_silu(rbf(g))), ox_f2bf(u));
  }
}

/* A call with n >= 2 tokens at key_dim 128 (text-dispatch -> text-batch,
 * prefill.rs:36-653): every layer runs over all tokens before the next
 * (batch.layer.fold), with the per-token operations of the decode step
 * where the batched kernels keep them (RMSNorm per row, qwen35.hex:912-977;
 * conv + L2 with history reads before the history commit,
 * batch_prepare.hex:3-292; the DeltaNet scan with the F32 state,
 * batch_scan.hex:1-200; gated norm, batch_gated.hex; head norm + RoPE + KV
 * append, batch_full_prepare.hex:3-97; staged attention per query,
 * batch_staged_attention.hex:10-47; router + select per token) and B256
 * projections for the rest. The recurrent state is imported into the F32
 * shadow before and persisted after (qwen35.hex:2-141); the head runs on the
 * last row (prefill.row). */
static int step_batch(ox_session* se, const uint64_t* tokens, int64_t n, int64_t start,
                      uint64_t* next_token, uint16_t* logits_out) {
  const ox_model* m = se->m;
  const ox_config* c = &m->c;
  const int64_t H = c->hidden, HD = c->head_dim, KVS = m->KVS, QS = m->QS;
  const int64_t KV_STRIDE = (int64_t)c->layers * 2 * KVS;
  const int64_t kv_end = se->capacity * KV_STRIDE;
  for (int l = 0; l < c->layers; ++l)
    for (int64_t i = 0; i < m->REC; ++i)
      se->shadow[l * m->REC + i] = ox_bf2f(se->cache[kv_end + l * m->LIN + m->CONV + i]);
  int64_t wide = m->QKV > 2 * QS ? m->QKV : 2 * QS;
  if (m->VS > wide) wide = m->VS;
  if (c->intermediate > wide) wide = c->intermediate;
  if (H > wide) wide = H;
  uint16_t* h = (uint16_t*)malloc(2 * (size_t)(n * H));
  uint16_t* x = (uint16_t*)malloc(2 * (size_t)(n * H));
  uint16_t* attn = (uint16_t*)malloc(2 * (size_t)(n * H));
  uint16_t* b1 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* b2 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* b3 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* b4 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* b5 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* b6 = (uint16_t*)malloc(2 * (size_t)(n * wide));
  uint16_t* row = (uint16_t*)malloc(2 * (size_t)wide);
  float rope[1024];
  for (int64_t t = 0; t < n; ++t)
    memcpy(h + t * H, (const uint16_t*)m->w[0] + tokens[t] * H, 2 * (size_t)H);  /* prefill.embed */
  for (int l = 0; l < c->layers; ++l) {
    const int64_t key_off = (int64_t)l * 2 * se->capacity * KVS;
    const int64_t value_off = key_off + se->capacity * KVS;
    normalize_rows(h, WF(m, l, 0), H, n, c->eps, x);
    int ffn;
    const float* post_norm;
    if (is_full(c, l)) {
      uint16_t *qg = b1, *kraw = b2, *vraw = b3, *qn = b4, *qr = b5, *ctx = b6;
      bproject(x, n, WB(m, l, 1), 2 * QS, H, qg);
      bproject(x, n, WB(m, l, 2), KVS, H, kraw);
      bproject(x, n, WB(m, l, 3), KVS, H, vraw);
      for (int64_t t = 0; t < n; ++t) {
        const int64_t position = start + t;
        uint16_t* qgt = qg + t * 2 * QS;
        uint16_t* kt = kraw + t * KVS;
        for (int hh = 0; hh < c->q_heads; ++hh)
          memcpy(qn + hh * HD, qgt + 2 * hh * HD, 2 * (size_t)HD);
        normalize_rows(qn, WF(m, l, g_plant == OX_PLANT_QK_NORM_SWAP ? 6 : 5), HD, c->q_heads, c->eps, qn);
        normalize_rows(kt, WF(m, l, g_plant == OX_PLANT_QK_NORM_SWAP ? 5 : 6), HD, c->kv_heads, c->eps, kt);
        rope_table(m, position, rope);
        for (int hh = 0; hh < c->q_heads; ++hh)
          rotate_head(qn + hh * HD, rope, (int)HD, c->rope_dim, qr + t * QS + hh * HD);
        for (int hh = 0; hh < c->kv_heads; ++hh)
          rotate_head(kt + hh * HD, rope, (int)HD, c->rope_dim,
                      se->cache + key_off + position * KVS + hh * HD);
        memcpy(se->cache + value_off + position * KVS, vraw + t * KVS, 2 * (size_t)KVS);
      }
      for (int64_t t = 0; t < n; ++t)
        attention_staged(m, qr + t * QS, se->cache, key_off, value_off, start + t + 1,
                         qg + t * 2 * QS, ctx + t * QS);
      bresidual(ctx, n, WB(m, l, 4), H, QS, h, attn);
      post_norm = WF(m, l, 7);
      ffn = 8;
    } else {
      uint16_t *qkv = b1, *z = b2, *ab = b3, *conv = b4, *core = b5, *gated = b6;
      const int64_t VH = c->value_heads;
      uint16_t* alpha = ab;
      uint16_t* beta = ab + n * VH;
      bproject(x, n, WB(m, l, 1), m->QKV, H, qkv);
      bproject(x, n, WB(m, l, 2), m->VS, H, z);
      bproject(x, n, WB(m, l, 3), VH, H, alpha);
      bproject(x, n, WB(m, l, 4), VH, H, beta);
      const int64_t conv_base = kv_end + l * m->LIN;
      for (int64_t t = 0; t < n; ++t) {
        uint16_t* ct = conv + t * m->QKV;
        conv_step(m, se->cache, conv_base, start + t, WF(m, l, 9), qkv + t * m->QKV, ct);
        uint16_t* q = row;
        uint16_t* k = row + m->KS;
        l2_heads(ct, c->key_heads, c->key_dim, q);
        l2_heads(ct + m->KS, c->key_heads, c->key_dim, k);
        delta_step(m, ct, q, k, alpha + t * VH, beta + t * VH, WF(m, l, 5), WF(m, l, 6), NULL,
                   se->shadow + l * m->REC, core + t * m->VS);
        gated_norm(m, core + t * m->VS, z + t * m->VS, WF(m, l, 7), gated + t * m->VS);
      }
      bresidual(gated, n, WB(m, l, 8), H, m->VS, h, attn);
      post_norm = WF(m, l, 10);
      ffn = 11;
    }
    normalize_rows(attn, post_norm, H, n, c->eps, x);
    if (c->moe) {
      for (int64_t t = 0; t < n; ++t)
        moe_ffn(m, se, l, ffn, x + t * H, attn + t * H, 1, h + t * H);
    } else {
      uint16_t* act = b1;
      bgate(x, n, WB(m, l, ffn + 0), WB(m, l, ffn + 1), c->intermediate, H, act);
      bresidual(act, n, WB(m, l, ffn + 2), H, c->intermediate, attn, h);
    }
  }
  for (int l = 0; l < c->layers; ++l)
    for (int64_t i = 0; i < m->REC; ++i)
      se->cache[kv_end + l * m->LIN + m->CONV + i] = ox_f2bf(se->shadow[l * m->REC + i]);
  int64_t total = ox_weight_count(c);
  normalize_rows(h + (n - 1) * H, (const float*)m->w[total - 2], H, 1, c->eps, x);
  uint16_t* logits = logits_out ? logits_out : (uint16_t*)malloc(2 * (size_t)c->vocab);
  project(x, (const uint16_t*)m->w[total - 1], c->vocab, H, 32, logits);
  argmax_bf16(logits, c->vocab, next_token);
  if (!logits_out) free(logits);
  free(h); free(x); free(attn); free(b1); free(b2); free(b3); free(b4); free(b5); free(b6);
  free(row);
  return 0;
}

int ox_step(ox_session* se, const uint64_t* tokens, int64_t n, int64_t start,
            uint64_t* next_token, uint16_t* logits_out) {
  const ox_model* m = se->m;
  const ox_config* c = &m->c;
  if (n < 1 || start < 0 || start + n > se->capacity || !attention_interval_ok(c)) return -1;
  for (int64_t t = 0; t < n; ++t)
    if (tokens[t] >= (uint64_t)c->vocab) return -2;
  if (n >= 2 && c->key_dim == 128)  /* text-dispatch, prefill.rs:623-652 */
    return step_batch(se, tokens, n, start, next_token, logits_out);
  const int64_t H = c->hidden, HD = c->head_dim, KVS = m->KVS, QS = m->QS;
  const int64_t KV_STRIDE = (int64_t)c->layers * 2 * KVS;
  const int64_t kv_end = se->capacity * KV_STRIDE;
  /* Dense: import the BF16 recurrent state into the F32 shadow every call;
   * MoE: only for multi-token calls (qwen35.hex:2-71; cached_delta.hex:189-228). */
  int shadow_mode = !c->moe || n >= 2;
  if (shadow_mode)
    for (int l = 0; l < c->layers; ++l)
      for (int64_t i = 0; i < m->REC; ++i)
        se->shadow[l * m->REC + i] = ox_bf2f(se->cache[kv_end + l * m->LIN + m->CONV + i]);

  size_t big = (size_t)(m->QKV > QS * 2 ? m->QKV : QS * 2);
  if ((size_t)H > big) big = (size_t)H;
  if ((size_t)m->VS > big) big = (size_t)m->VS;
  if ((size_t)c->intermediate > big) big = (size_t)c->intermediate;
  uint16_t* h = (uint16_t*)malloc(2 * (size_t)H);
  uint16_t* x = (uint16_t*)malloc(2 * (size_t)H);
  uint16_t* attn = (uint16_t*)malloc(2 * (size_t)H);
  uint16_t* b1 = (uint16_t*)malloc(2 * big);
  uint16_t* b2 = (uint16_t*)malloc(2 * big);
  uint16_t* b3 = (uint16_t*)malloc(2 * big);
  uint16_t* b4 = (uint16_t*)malloc(2 * big);
  uint16_t* b5 = (uint16_t*)malloc(2 * big);
  uint16_t* b6 = (uint16_t*)malloc(2 * big);
  float rope[1024];
  for (int64_t t = 0; t < n; ++t) {
    int64_t position = start + t;
    memcpy(h, (const uint16_t*)m->w[0] + tokens[t] * H, 2 * (size_t)H);  /* embedding.hex:5-14 */
    rope_table(m, position, rope);
    for (int l = 0; l < c->layers; ++l) {
      int64_t key_off = (int64_t)l * 2 * se->capacity * KVS;
      int64_t value_off = key_off + se->capacity * KVS;
      normalize_rows(h, WF(m, l, 0), H, 1, c->eps, x);
      int ffn;
      const float* post_norm;
      if (is_full(c, l)) {
        /* qg = [q|gate] per head; k; v (group-project S256 for MoE,
         * fused.project S32 for dense: qwen35.rs:366-381, 571). */
        int width = c->moe ? 256 : 32;
        uint16_t *qg = b1, *kraw = b2, *vraw = b3, *qn = b4, *qr = b5, *ctx = b6;
        project(x, WB(m, l, 1), 2 * QS, H, width, qg);
        project(x, WB(m, l, 2), KVS, H, width, kraw);
        project(x, WB(m, l, 3), KVS, H, width, vraw);
        for (int hh = 0; hh < c->q_heads; ++hh)
          memcpy(qn + hh * HD, qg + 2 * hh * HD, 2 * (size_t)HD);  /* qwen35.query */
        normalize_rows(qn, WF(m, l, g_plant == OX_PLANT_QK_NORM_SWAP ? 6 : 5), HD, c->q_heads, c->eps, qn);
        normalize_rows(kraw, WF(m, l, g_plant == OX_PLANT_QK_NORM_SWAP ? 5 : 6), HD, c->kv_heads, c->eps, kraw);
        for (int hh = 0; hh < c->q_heads; ++hh)
          rotate_head(qn + hh * HD, rope, (int)HD, c->rope_dim, qr + hh * HD);
        for (int hh = 0; hh < c->kv_heads; ++hh)
          rotate_head(kraw + hh * HD, rope, (int)HD, c->rope_dim,
                      se->cache + key_off + position * KVS + hh * HD);
        memcpy(se->cache + value_off + position * KVS, vraw, 2 * (size_t)KVS);
        if (c->moe)
          attention_online(m, qr, se->cache, key_off, value_off, position + 1, qg, se->split_keys, ctx);
        else
          attention_staged(m, qr, se->cache, key_off, value_off, position + 1, qg, ctx);
        residual_project(ctx, WB(m, l, 4), H, QS, h, attn);
        post_norm = WF(m, l, 7);
        ffn = 8;
      } else {
        int width = c->moe ? 256 : 32;
        uint16_t *qkv = b1, *z = b2, *conv = b3, *core = b4, *gated = b5;
        uint16_t alpha[1024], beta[1024];
        project(x, WB(m, l, 1), m->QKV, H, width, qkv);
        project(x, WB(m, l, 2), m->VS, H, width, z);
        project(x, WB(m, l, 3), c->value_heads, H, width, alpha);
        project(x, WB(m, l, 4), c->value_heads, H, width, beta);
        int64_t conv_base = kv_end + l * m->LIN;
        conv_step(m, se->cache, conv_base, position, WF(m, l, 9), qkv, conv);
        uint16_t* q = b6;
        uint16_t* k = b6 + m->KS;
        l2_heads(conv, c->key_heads, c->key_dim, q);
        l2_heads(conv + m->KS, c->key_heads, c->key_dim, k);
        if (shadow_mode)
          delta_step(m, conv, q, k, alpha, beta, WF(m, l, 5), WF(m, l, 6), NULL,
                     se->shadow + l * m->REC, core);
        else
          delta_step(m, conv, q, k, alpha, beta, WF(m, l, 5), WF(m, l, 6),
                     se->cache + conv_base + m->CONV, NULL, core);
        gated_norm(m, core, z, WF(m, l, 7), gated);
        residual_project(gated, WB(m, l, 8), H, m->VS, h, attn);
        post_norm = WF(m, l, 10);
        ffn = 11;
      }
      normalize_rows(attn, post_norm, H, 1, c->eps, x);
      if (c->moe) {
        moe_ffn(m, se, l, ffn, x, attn, 0, h);
      } else {
        uint16_t* act = b1;
        swiglu_project(x, WB(m, l, ffn + 0), WB(m, l, ffn + 1), c->intermediate, H, act);
        residual_project(act, WB(m, l, ffn + 2), H, c->intermediate, attn, h);
      }
    }
  }
  if (shadow_mode)  /* persist: F32 shadow -> BF16 cache (qwen35.hex:72-141) */
    for (int l = 0; l < c->layers; ++l)
      for (int64_t i = 0; i < m->REC; ++i)
        se->cache[kv_end + l * m->LIN + m->CONV + i] = ox_f2bf(se->shadow[l * m->REC + i]);
  /* head: normalize, S32 vocab projection, argmax (qwen35.rs:1612-1632). */
  int64_t total = ox_weight_count(c);
  normalize_rows(h, (const float*)m->w[total - 2], H, 1, c->eps, x);
  uint16_t* logits = logits_out ? logits_out : (uint16_t*)malloc(2 * (size_t)c->vocab);
  project(x, (const uint16_t*)m->w[total - 1], c->vocab, H, 32, logits);
  argmax_bf16(logits, c->vocab, next_token);
  if (!logits_out) free(logits);
  free(h); free(x); free(attn); free(b1); free(b2); free(b3); free(b4); free(b5); free(b6);
  return 0;
}

void ox_set_threads(int n) {
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#else
  (void)n;
#endif
}

/* ----------------------------------------------- kernel-level entry points
 * (for the known-answer tests of tests/qwen35_simt.rs:129-434). */
void ox_project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols, int width,
                uint16_t* out) {
  project(x, w, rows, cols, width, out);
}
void ox_residual_project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols,
                         const uint16_t* residual, uint16_t* out) {
  residual_project(x, w, rows, cols, residual, out);
}
void ox_swiglu_project(const uint16_t* x, const uint16_t* wg, const uint16_t* wu, int64_t rows,
                       int64_t cols, uint16_t* out) {
  swiglu_project(x, wg, wu, rows, cols, out);
}
/* MoE gate/up and down with explicit ids/probs (moe.hex:254-434). */
void ox_moe_gate_rows(const uint16_t* x, const uint16_t* gate, const uint16_t* up,
                      const uint16_t* sgate, const uint16_t* sup, const int64_t* ids,
                      const float* probs, float shared_logit, int64_t H, int64_t K, int64_t I,
                      int64_t SI, uint16_t* active) {
  const float shared_prob = ox_sigmoid(shared_logit);
  for (int64_t r = 0; r < K * I + SI; ++r) {
    int routed = r < K * I;
    const uint16_t *wg, *wu;
    int64_t slot = 0;
    if (routed) {
      slot = r / I;
      int64_t row = ids[slot] * I + r % I;
      wg = gate + row * H; wu = up + row * H;
    } else {
      wg = sgate + (r - K * I) * H; wu = sup + (r - K * I) * H;
    }
    float g, u;
    dot_dual(x, wg, wu, H / 2, 256, &g, &u);
    float gb = rbf(g), ub = rbf(u);
    float activated = ox_silu(gb);
    float y = routed ? (activated * ub) * probs[slot] : rbf(rbf(activated) * ub) * shared_prob;
    active[r] = ox_f2bf(y);
  }
}
void ox_moe_down_rows(const uint16_t* active, const uint16_t* down, const uint16_t* sdown,
                      const int64_t* ids, const uint16_t* residual, int64_t H, int64_t K,
                      int64_t I, int64_t SI, uint16_t* out) {
  const int64_t ip = I / 2, ap = K * I / 2, sp = SI / 2;
  for (int64_t o = 0; o < H; ++o) {
    float lanes[32];
    for (int lane = 0; lane < 32; ++lane) {
      float lo = 0.0f, hi = 0.0f;
      for (int64_t p = lane; p < ap; p += 32) {
        const uint16_t* w = down + (ids[p / ip] * H + o) * I + 2 * (p % ip);
        lo += ox_bf2f(active[2 * p]) * ox_bf2f(w[0]);
        hi += ox_bf2f(active[2 * p + 1]) * ox_bf2f(w[1]);
      }
      lanes[lane] = lo + hi;
    }
    float routed = tree(lanes, 32);
    float shared = ox_dot_width(active + K * I, sdown + o * SI, sp, 32);
    out[o] = bf_add(ox_f2bf(routed + ox_bf2f(residual[o])), ox_f2bf(shared));
  }
}
/* Router logits + top-k selection (moe.hex:4-252). */
void ox_moe_route(const uint16_t* x, const float* router, const float* shared_router, int64_t H,
                  int64_t E, int64_t K, float* logits, int64_t* ids, float* probs) {
  for (int64_t e = 0; e <= E; ++e)
    logits[e] = ox_dot_width_f32w(x, e < E ? router + e * H : shared_router, H / 2, 32);
  select_top_k(logits, E, K, ids, probs);
}

/* ------------------------------------------ kernel-level entry points */
/* One restated function each, on explicit buffers, for the per-function
 * pins (tests/test_oracle_pins.py); dims come from the model's config. */

void ox_k_normalize(const uint16_t* x, const float* w, int64_t cols, int64_t rows, float eps,
                    uint16_t* out) {
  normalize_rows(x, w, cols, rows, eps, out);
}

/* Head RMS norm with weights w (full_prepare.hex:20-48) then RoPE at
 * `position` (rope.hex:5-82), for `heads` heads of head_dim. */
void ox_k_prepare_heads(const ox_model* m, int64_t position, const uint16_t* in, const float* w,
                        int64_t heads, uint16_t* out) {
  const int HD = m->c.head_dim;
  uint16_t* tmp = (uint16_t*)malloc(2 * (size_t)(heads * HD));
  float rope[1024];
  normalize_rows(in, w, HD, heads, m->c.eps, tmp);
  rope_table(m, position, rope);
  for (int64_t h = 0; h < heads; ++h) rotate_head(tmp + h * HD, rope, HD, m->c.rope_dim, out + h * HD);
  free(tmp);
}

/* RoPE alone on already normalised heads. */
void ox_k_rope(const ox_model* m, int64_t position, const uint16_t* in, int64_t heads, uint16_t* out) {
  const int HD = m->c.head_dim;
  float rope[1024];
  rope_table(m, position, rope);
  for (int64_t h = 0; h < heads; ++h) rotate_head(in + h * HD, rope, HD, m->c.rope_dim, out + h * HD);
}

/* Conv over a 3-slot history [3][QKV] (updated in place). */
void ox_k_conv(const ox_model* m, uint16_t* history, int64_t position, const float* weight,
               const uint16_t* qkv, uint16_t* out) {
  conv_step(m, history, 0, position, weight, qkv, out);
}

void ox_k_l2(const uint16_t* in, int heads, int dim, uint16_t* out) { l2_heads(in, heads, dim, out); }

void ox_k_delta(const ox_model* m, const uint16_t* conv, const uint16_t* q, const uint16_t* k,
                const uint16_t* alpha, const uint16_t* beta, const float* dt, const float* a,
                uint16_t* state16, float* state32, uint16_t* out) {
  delta_step(m, conv, q, k, alpha, beta, dt, a, state16, state32, out);
}

void ox_k_gated_norm(const ox_model* m, const uint16_t* core, const uint16_t* z, const float* w,
                     uint16_t* out) {
  gated_norm(m, core, z, w, out);
}

/* Top-k selection alone, over given router logits (moe.hex:86-252). */
void ox_k_select(const float* logits, int64_t E, int64_t K, int64_t* ids, float* probs) {
  select_top_k(logits, E, K, ids, probs);
}

/* Greedy argmax over BF16 logits (fused_argmax.hex:1-205). */
uint64_t ox_k_argmax(const uint16_t* logits, int64_t vocab) {
  uint64_t t = 0;
  argmax_bf16(logits, vocab, &t);
  return t;
}

/* Decode attention over `keys` cached rows: kv = [keys][KVS] keys then
 * [keys][KVS] values; online (MoE decode) or staged (dense). */
void ox_k_attention(const ox_model* m, int online, const uint16_t* q, const uint16_t* kv, int64_t keys,
                    const uint16_t* qg, int64_t split_keys, uint16_t* out) {
  if (online) attention_online(m, q, kv, 0, keys * m->KVS, keys, qg, split_keys, out);
  else attention_staged(m, q, kv, 0, keys * m->KVS, keys, qg, out);
}
