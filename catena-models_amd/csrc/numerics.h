// Scalar numerics of the token loop, compiled for both gfx950 and the host.
//
// Every function is written with ordinary IEEE binary32 operations and the
// library is built with -ffp-contract=off, so each multiply and add rounds
// separately (the reference's contract, src/catena/numeric.hex:10). Division
// is the correctly rounded one (-fhip-fp32-correctly-rounded-divide-sqrt).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define CQ35_HD __host__ __device__ __forceinline__

namespace cq35 {

CQ35_HD uint32_t fbits(float x) { return __builtin_bit_cast(uint32_t, x); }
CQ35_HD float bitsf(uint32_t u) { return __builtin_bit_cast(float, u); }

// F32 -> BF16, nearest-even, NaNs quieted (src/weights.rs:213-221).
// On the device one v_cvt_pk_bf16_f32 (denormals kept: the library is built
// without flushing), equal to the integer formula below for every one of the
// 2^32 inputs (checked exhaustively on MI355X; tests/test_gpu_parity.py
// checks every exponent, sign and NaN class); the host uses the formula.
CQ35_HD uint16_t f2bf(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_bit_cast(uint16_t, (__bf16)x);
#else
  const uint32_t u = fbits(x);
  const uint32_t quiet = (u >> 16) | 0x0040u;
  const uint32_t rounded = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  return (uint16_t)(x != x ? quiet : rounded);
#endif
}
CQ35_HD float bf2f(uint16_t b) { return bitsf((uint32_t)b << 16); }
CQ35_HD float rbf(float x) { return bf2f(f2bf(x)); }
// Low / high BF16 halves of a packed pair, widened (bf16x2.low/high).
CQ35_HD float lo2f(uint32_t p) { return bitsf(p << 16); }
CQ35_HD float hi2f(uint32_t p) { return bitsf(p & 0xffff0000u); }
// bf16.add / bf16.mul: widen, operate in F32, round (memory.hex:920-935).
CQ35_HD uint16_t bf_add(uint16_t a, uint16_t b) { return f2bf(bf2f(a) + bf2f(b)); }
CQ35_HD uint16_t bf_mul(uint16_t a, uint16_t b) { return f2bf(bf2f(a) * bf2f(b)); }

// Nearest integer of a non-negative F32, ties away from zero.
CQ35_HD uint32_t round_u32(float x) {
  float t = __builtin_truncf(x);
  if (x - t >= 0.5f) t += 1.0f;
  return (uint32_t)t;
}

// Scaling by 2^n through the exponent bits, with nearest-even rounding into
// the subnormal range (numeric.hex:30-61).
CQ35_HD float exp_scale(float y, uint32_t n, bool negative) {
  const uint32_t yb = fbits(y);
  const uint32_t exponent = yb >> 23;
  const bool subnormal = exponent <= n;
  const uint32_t shift = subnormal ? (n - exponent) + 1u : 1u;
  const uint32_t significand = (yb & 0x007fffffu) + 0x00800000u;
  const uint32_t truncated = significand >> shift;
  const uint32_t power = 0x80000000u >> (31u - shift);
  const uint32_t remainder = significand - truncated * power;
  const uint32_t half = power >> 1;
  const bool round_up = (half < remainder) || (half == remainder && (truncated & 1u));
  const uint32_t sub_bits = truncated + (round_up ? 1u : 0u);
  const uint32_t offset = n * 0x00800000u;
  return bitsf(negative ? (subnormal ? sub_bits : yb - offset) : yb + offset);
}

// fdlibm-style F32 exponential (numeric.hex:63-102): split ln2 reduction,
// rational correction, integer rescaling.
CQ35_HD float hexp(float x) {
  const uint32_t bits = fbits(x);
  const uint32_t magnitude = bits & 0x7fffffffu;
  const bool negative = bits >= 0x80000000u;
  const bool nan = magnitude > 0x7f800000u;
  const bool finite_range = magnitude < (negative ? 0x42cff1b5u : 0x42b17218u);
  const float safe_x = finite_range ? x : 0.0f;
  const float absolute = negative ? -safe_x : safe_x;
  const uint32_t n = round_u32(absolute * bitsf(0x3fb8aa3bu));
  const float nf = (float)n;
  const float k = negative ? -nf : nf;
  const float hi = safe_x - k * bitsf(0x3f317200u);
  const float lo = k * bitsf(0x35bfbe8eu);
  const float r = hi - lo;
  const float square = r * r;
  const float polynomial = bitsf(0x3e2aaa8fu) + square * bitsf(0xbb355215u);
  const float c = r - square * polynomial;
  const float ratio = (r * c) / (2.0f - c);
  const float y = 1.0f - ((lo - ratio) - hi);
  const float scaled = exp_scale(y, n, negative);
  const float finite = magnitude < 0x39000000u ? 1.0f + safe_x : scaled;
  const float classified = finite_range ? finite : (negative ? 0.0f : bitsf(0x7f800000u));
  return nan ? bitsf(0x7fc00000u) : classified;
}

CQ35_HD float silu(float x) { return x / (1.0f + hexp(-x)); }      // numeric.hex:104-113
CQ35_HD float sigmoid(float x) { return 1.0f / (1.0f + hexp(-x)); } // numeric.hex:115-124

// max(x, 0) + 2 atanh(e / (2 + e)), e = exp(-|x|) (numeric.hex:126-174).
CQ35_HD float softplus(float x) {
  const bool positive = x > 0.0f;
  const float maximum = positive ? x : 0.0f;
  const float e = hexp(positive ? -x : x);
  const float z = e / (2.0f + e);
  const float z2 = z * z;
  float p = bitsf(0x3d888889u) + z2 * bitsf(0x3d70f0f1u);
  p = bitsf(0x3d9d89d9u) + z2 * p;
  p = bitsf(0x3dba2e8cu) + z2 * p;
  p = bitsf(0x3de38e39u) + z2 * p;
  p = bitsf(0x3e124925u) + z2 * p;
  p = bitsf(0x3e4ccccdu) + z2 * p;
  p = bitsf(0x3eaaaaabu) + z2 * p;
  p = 1.0f + z2 * p;
  return maximum + 2.0f * (z * p);
}

// Exponent-halving initial guess and four Newton steps (numeric.hex:176-206).
CQ35_HD float nsqrt(float x) {
  float g = bitsf((fbits(x) >> 1) + 0x1fc00000u);
  g = (g + x / g) * 0.5f;
  g = (g + x / g) * 0.5f;
  g = (g + x / g) * 0.5f;
  g = (g + x / g) * 0.5f;
  return x <= 0.0f ? 0.0f : g;
}

// Three-part pi/2 reduction and degree-13/14 polynomials (numeric.hex:208-287).
CQ35_HD void sincos_q(float angle, float* sine, float* cosine) {
  const uint32_t q = round_u32(angle * bitsf(0x3f22f983u));
  const float qf = (float)q;
  float r = angle - qf * bitsf(0x3fc90000u);
  r = r - qf * bitsf(0x39fda000u);
  r = r - qf * bitsf(0x33a22169u);
  const float s2 = r * r;
  float sp = bitsf(0xb2d72f34u) + s2 * bitsf(0x2f2ec9d3u);
  sp = bitsf(0x3638ef1bu) + s2 * sp;
  sp = bitsf(0xb9500d01u) + s2 * sp;
  sp = bitsf(0x3c088889u) + s2 * sp;
  sp = bitsf(0xbe2aaaabu) + s2 * sp;
  const float s = r + (r * s2) * sp;
  float cp = bitsf(0x310f74f6u) + s2 * bitsf(0xad47d74eu);
  cp = bitsf(0xb493f27cu) + s2 * cp;
  cp = bitsf(0x37d00d01u) + s2 * cp;
  cp = bitsf(0xbab60b61u) + s2 * cp;
  cp = bitsf(0x3d2aaaabu) + s2 * cp;
  const float c = (1.0f - s2 * 0.5f) + (s2 * s2) * cp;
  switch (q & 3u) {
    case 0: *sine = s; *cosine = c; break;
    case 1: *sine = c; *cosine = -s; break;
    case 2: *sine = -s; *cosine = -c; break;
    default: *sine = -c; *cosine = s; break;
  }
}

// Synthetic weight generator (the bench/test checkpoint): SplitMix64
// finaliser keyed by (seed, tensor), counted by element; the centred sum of
// the four 16-bit fields approximates a normal variate (Irwin-Hall, n = 4).
CQ35_HD uint64_t mix64(uint64_t x) {
  x ^= x >> 30; x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27; x *= 0x94d049bb133111ebull;
  x ^= x >> 31;
  return x;
}
CQ35_HD int32_t irwin_hall4(uint64_t h) {
  return (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
         (int32_t)(h >> 48) - 131070;
}

}  // namespace cq35
