// Decode attention over the BF16 KV cache in the reference's exact order
// (qwen35_online.hex:4-331), split into two launches so the work spreads over
// the chip instead of one block per query head:
//
//  k_attn_scores  every (key, KV head) in parallel: 32-lane dots (lane l owns
//                 channels l, l+32, ..., serial from 0.0, then a 32-wide
//                 halving tree) for all query heads sharing the KV head, x
//                 1/sqrt(HD);
//  k_attn_values  per (query head, 16-channel chunk): running maximum per
//                 8-key tile (a prefix maximum of the tile maxima: max is
//                 exact), alpha_t = exp(m_{t-1} - m_t) and p = exp(s - m_t) in
//                 parallel, then each channel's serial chain
//                 acc = acc*alpha_t + p_0 v_0 + ... + p_7 v_7 while a helper
//                 lane runs the denominator chain den = den*alpha_t + p_0 + ...;
//                 out = bf16(bf16(acc/den) * sigmoid(gate)).
//
// Both chains keep the reference's tile structure (8 keys, invalid keys
// contribute p = 0 against key 0's value), so the result is bit-identical.
#pragma once

#include "layers.h"

namespace cq35 {

constexpr int kScoreBlock = 256;  // 8 key units of 32 lanes

// rows != nullptr: grid z is the session of a batched step (its cache,
// position, query rows [z][q_heads * head_dim] and scores [z][q_heads][stride]).
__global__ __launch_bounds__(kScoreBlock) void k_attn_scores(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ cache, int64_t key_base,
    const uint64_t* __restrict__ params, int t, int kvs, int head_dim, int heads_per_kv,
    float scale, float* __restrict__ scores, int stride, const SessionRows* __restrict__ rows) {
  extern __shared__ float qs[];  // heads_per_kv * head_dim
  const int kvh = blockIdx.y, tid = threadIdx.x;
  int64_t keys;
  if (rows) {
    const int b = blockIdx.z;
    const int q_heads = gridDim.y * heads_per_kv;
    keys = (int64_t)rows->position[b] + 1;
    cache = rows->cache[b];
    q += (size_t)b * q_heads * head_dim;
    scores += (size_t)b * q_heads * stride;
  } else {
    keys = (int64_t)params[0] + t + 1;
  }
  const int nq = heads_per_kv * head_dim;
  for (int i = tid; i < nq; i += kScoreBlock) qs[i] = bf2f(q[(size_t)kvh * nq + i]);
  __syncthreads();
  const int unit = tid >> 5, lane = tid & 31;
  const int steps = head_dim >> 5;
  const uint16_t* kbase = cache + key_base + (int64_t)kvh * head_dim + lane;
  for (int64_t kk = (int64_t)blockIdx.x * 8 + unit; kk < keys; kk += (int64_t)gridDim.x * 8) {
    const uint16_t* kr = kbase + kk * kvs;
    float kv[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) kv[j] = j < steps ? bf2f(kr[32 * j]) : 0.0f;
    for (int h = 0; h < heads_per_kv; ++h) {
      const float* qh = qs + h * head_dim + lane;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < steps) acc += qh[32 * j] * kv[j];
#pragma unroll
      for (int s = 16; s >= 1; s >>= 1) acc += __shfl_down(acc, s, 32);
      if (lane == 0) scores[(size_t)(kvh * heads_per_kv + h) * stride + kk] = acc * scale;
    }
  }
}

// One wave per (query head, 16-channel chunk). Keys are processed in chunks
// of up to kValueChunk: the wave stages the chunk's V slice into LDS with
// 16-byte loads (all in flight at once) and computes the chunk's weights,
// then lanes 0-15 run the channel chains from LDS (the other lanes repeat
// them) and every lane the denominator chain.
//
// Split-K above split_keys keys (0: never): the T tiles form at most
// kSplitRanges ranges of ceil(T / kSplitRanges) tiles (the ranges depend on
// the key count only) and each range runs the online recurrence from
// scratch over its own tiles (running maximum reset at the range start, so
// its first alpha is 0); at each range's end its accumulators join the
// totals in ascending range order weighted by w_r = exp(m_r - M), M the
// maximum over all scores: den = 0 + den_0 w_0 + den_1 w_1 + ..., each
// channel likewise. At or below the threshold one chain runs over all tiles,
// the reference's, bit for bit.
constexpr int kValueChannels = 16;
constexpr int kValueChunk = 1024;
constexpr int kSplitRanges = 128;

__global__ __launch_bounds__(64) void k_attn_values(
    const float* __restrict__ scores, int stride, const uint16_t* __restrict__ cache,
    int64_t value_base, const uint64_t* __restrict__ params, int t, int kvs, int head_dim,
    int heads_per_kv, const uint16_t* __restrict__ qg, int64_t split_keys, uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) float lds[];
  const int head = blockIdx.x, chunk = blockIdx.y, lane = threadIdx.x;
  const int64_t keys = (int64_t)params[0] + t + 1;
  const int tiles = (int)((keys + 7) >> 3);
  const bool split = split_keys > 0 && keys > split_keys;
  const int range_tiles = split ? (tiles + kSplitRanges - 1) / kSplitRanges : tiles;
  float* mx = lds;                                   // running maximum per tile (all tiles)
  float* p = mx + ((tiles + 3) & ~3);                // weights of the current key chunk
  float* alpha = p + kValueChunk;                    // exp(m_prev - m_t) of the chunk
  u32x4* vs = reinterpret_cast<u32x4*>(alpha + kValueChunk / 8);  // [chunk keys][16 ch] bf16
  const float* s = scores + (size_t)head * stride;
  const float ninf = bitsf(0xff800000u);
  for (int i = lane; i < tiles; i += 64) {
    float m = ninf;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t k = (int64_t)i * 8 + j;
      m = fmaxf(m, k < keys ? s[k] : ninf);
    }
    mx[i] = m;
  }
  __syncthreads();
  float top = ninf;  // the maximum of all scores (lane 0)
  if (lane == 0) {
    float m = ninf;
    for (int i = 0; i < tiles; ++i) {
      if (split && i % range_tiles == 0) m = ninf;
      m = fmaxf(m, mx[i]);
      mx[i] = m;
      top = fmaxf(top, m);
    }
  }
  __syncthreads();
  top = __shfl(top, 0, 64);
  const int c0 = chunk * kValueChannels;
  const uint16_t* vbase = cache + value_base + (int64_t)(head / heads_per_kv) * head_dim + c0;
  float acc = 0.0f, den = 0.0f, acc_all = 0.0f, den_all = 0.0f;
  for (int64_t k0 = 0; k0 < (int64_t)tiles * 8; k0 += kValueChunk) {
    const int n = (int)min<int64_t>(kValueChunk, (int64_t)tiles * 8 - k0);  // multiple of 8
    // stage V rows k0..k0+n (16 channels = 2 quads per key; invalid keys read key 0)
#pragma unroll 8
    for (int i = lane; i < 2 * n; i += 64) {
      const int64_t k = k0 + (i >> 1);
      const int64_t safe = k < keys ? k : 0;
      vs[i] = reinterpret_cast<const u32x4*>(vbase + safe * kvs)[i & 1];
    }
    for (int i = lane; i < n; i += 64) {
      const int64_t k = k0 + i;
      p[i] = k < keys ? hexp(s[k] - mx[k >> 3]) : 0.0f;
    }
    for (int i = lane; i < n / 8; i += 64) {
      const int tile = (int)(k0 / 8) + i;
      const bool first = tile == 0 || (split && tile % range_tiles == 0);
      alpha[i] = hexp((first ? ninf : mx[tile - 1]) - mx[tile]);
    }
    __syncthreads();
    const uint16_t* vh = reinterpret_cast<const uint16_t*>(vs) + (lane & 15);
    for (int i = 0; i < n / 8; ++i) {
      acc = acc * alpha[i];
      den = den * alpha[i];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        acc = acc + p[i * 8 + j] * bf2f(vh[(i * 8 + j) * kValueChannels]);
        den = den + p[i * 8 + j];
      }
      const int tile = (int)(k0 / 8) + i;
      if (split && (tile % range_tiles == range_tiles - 1 || tile == tiles - 1)) {
        const float w = hexp(mx[tile] - top);  // the range's running maximum at its last tile
        acc_all = acc_all + acc * w;
        den_all = den_all + den * w;
        acc = 0.0f;  // the next range starts from zero
        den = 0.0f;
      }
    }
    __syncthreads();
  }
  if (split) {
    acc = acc_all;
    den = den_all;
  }
  const int c = c0 + lane;
  if (lane < kValueChannels && c < head_dim) {
    const float gate = sigmoid(bf2f(qg[(size_t)head * 2 * head_dim + head_dim + c]));
    out[head * head_dim + c] = f2bf(rbf(acc / den) * gate);
  }
}

inline size_t attn_values_lds_bytes(int64_t capacity) {
  const int64_t tiles = (capacity + 7) / 8;
  return (size_t)((tiles + 3) / 4 * 4 + kValueChunk + kValueChunk / 8) * sizeof(float) +
         (size_t)kValueChunk * kValueChannels * 2;
}

}  // namespace cq35
