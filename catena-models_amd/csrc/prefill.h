// Batched prefill: the reference's multi-token path for key_dim 128
// (text-dispatch -> text-batch, prefill.rs:36-653). Every layer runs over all
// tokens of a chunk before the next layer. Per-token operations keep the
// decode arithmetic (they are the same reference programs with a token index):
// RMSNorm rows, convolution + L2 with history reads before the history commit,
// the DeltaNet scan over the F32 state, gated norm, head norm + RoPE + KV
// append, staged attention per query, router and top-k. The projections use
// the batched order B256: reference lane l (of 256) visits pairs l, l+256, ...
// with ONE accumulator, acc = (acc + x.lo*w.lo) + x.hi*w.hi
// (batch_projection.hex:4-18 with numeric.hex:17-28), then the 256-wide
// halving tree (cooperative.hex:285-335).
//
// Wave mapping of B256: physical lane q holds reference lanes 4q..4q+3, so
// its 16-byte quads q, q+64, q+128, ... are exactly those lanes' pairs in
// visiting order; reference strides 128..4 are physical strides 32..1
// (tree_levels<64>), strides 2 and 1 are in-lane.
#pragma once

#include "layers.h"

namespace cq35 {

constexpr int kBTokens = 8;   // tokens per wave sharing each weight quad
constexpr int kBChunk = 256;  // tokens per chunk (buffer rows)
constexpr int kMChunk = 1024;  // tokens per chunk with matrix-core components

__device__ __forceinline__ void b256_acc(float (&a)[4], const u32x4& x, const u32x4& w) {
  a[0] = (a[0] + lo2f(x.x) * lo2f(w.x)) + hi2f(x.x) * hi2f(w.x);
  a[1] = (a[1] + lo2f(x.y) * lo2f(w.y)) + hi2f(x.y) * hi2f(w.y);
  a[2] = (a[2] + lo2f(x.z) * lo2f(w.z)) + hi2f(x.z) * hi2f(w.z);
  a[3] = (a[3] + lo2f(x.w) * lo2f(w.w)) + hi2f(x.w) * hi2f(w.w);
}

// Tree over the 256 reference lanes; every lane of the wave must call it.
// The total is valid in lane 0.
__device__ __forceinline__ float b256_tree(const float (&a)[4]) {
  float v0 = a[0], v1 = a[1], v2 = a[2], v3 = a[3];
  tree_levels<64>(v0, v1, v2, v3);
  v0 += v2;
  v1 += v3;
  return v0 + v1;
}

// Two B256 trees at once (tree64_pair4_end: every sum with b256_tree's
// operands): a's total in lane 31, b's in lane 63.
__device__ __forceinline__ float b256_tree2(const float (&a)[4], const float (&b)[4]) {
  return tree64_pair4_end(a, b);
}

enum { kBPlain = 0, kBResidual = 1, kBGate = 2 };

// out[t][row] for `rows` outputs of `n` token rows of width `cols`
// (batch.project / batch.residual / batch.gate, batch_projection.hex:30-279,
// 280-530, 531-854). Block (bproject_rows rows, 32-token group): wave w takes
// tokens [32*by + 8w, +8) and shares each weight quad across them. Epilogues:
// bf16(total); bf16(bf16(total) (+) res); bf16(bf16(silu(bf16 g))) (x) bf16(u).
// Requires cols % 8 == 0.
// kBRows output rows per block (plain and residual modes: each wave takes
// them all, its token quads shared by the rows; gate mode: one row).
template <int kMode>
constexpr int bproject_rows() { return kMode == kBGate ? 1 : 2; }

template <int kMode>
__global__ __launch_bounds__(kBlock) void k_bproject(const uint16_t* __restrict__ x, int n,
                                                     int cols, const uint16_t* __restrict__ w,
                                                     const uint16_t* __restrict__ w2, int rows,
                                                     const uint16_t* __restrict__ res,
                                                     uint16_t* __restrict__ out) {
  constexpr int R = bproject_rows<kMode>();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * R;
  const int t0 = (blockIdx.y * 4 + wave) * kBTokens;
  if (t0 >= n || row0 >= rows) return;  // wave-uniform
  const int quads = cols >> 3;
  const u32x4* wr[R];
#pragma unroll
  for (int k = 0; k < R; ++k) wr[k] = reinterpret_cast<const u32x4*>(w + (size_t)min(row0 + k, rows - 1) * cols);
  const u32x4* wr2 = kMode == kBGate ? reinterpret_cast<const u32x4*>(w2 + (size_t)row0 * cols) : nullptr;
  float acc[R][kBTokens][4], acc2[kMode == kBGate ? kBTokens : 1][4];
#pragma unroll
  for (int t = 0; t < kBTokens; ++t)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
#pragma unroll
      for (int k = 0; k < R; ++k) acc[k][t][r] = 0.0f;
      if (kMode == kBGate) acc2[t][r] = 0.0f;
    }
  for (int qi = lane; qi < quads; qi += 64) {
    u32x4 wq[R];
#pragma unroll
    for (int k = 0; k < R; ++k) wq[k] = wr[k][qi];
    u32x4 wq2;
    if (kMode == kBGate) wq2 = wr2[qi];
#pragma unroll
    for (int t = 0; t < kBTokens; ++t) {
      if (t0 + t < n) {
        const u32x4 xq = reinterpret_cast<const u32x4*>(x + (size_t)(t0 + t) * cols)[qi];
#pragma unroll
        for (int k = 0; k < R; ++k) b256_acc(acc[k][t], xq, wq[k]);
        if (kMode == kBGate) b256_acc(acc2[kMode == kBGate ? t : 0], xq, wq2);
      }
    }
  }
  // totals: rows in pairs (or the gate and up sums) through b256_tree2
  float tot[R][kBTokens], tot2[kBTokens];
#pragma unroll
  for (int t = 0; t < kBTokens; ++t) {
    if (t0 + t >= n) break;  // wave-uniform
    if (kMode == kBGate) {
      const float both = b256_tree2(acc[0][t], acc2[kMode == kBGate ? t : 0]);
      tot[0][t] = lane_value(both, 31);
      tot2[t] = lane_value(both, 63);
    } else {
#pragma unroll
      for (int k = 0; k + 1 < R; k += 2) {
        const float both = b256_tree2(acc[k][t], acc[k + 1][t]);
        tot[k][t] = lane_value(both, 31);
        tot[k + 1][t] = lane_value(both, 63);
      }
      if (R % 2) tot[R - 1][t] = b256_tree(acc[R - 1][t]);
    }
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int row = row0 + k;
    if (row >= rows) break;  // wave-uniform
#pragma unroll
    for (int t = 0; t < kBTokens; ++t) {
      if (t0 + t >= n) break;  // wave-uniform
      const float total = tot[k][t];
      const float total2 = kMode == kBGate ? tot2[t] : 0.0f;
      if (lane == 0) {
        const size_t o = (size_t)(t0 + t) * rows + row;
        uint16_t y;
        if (kMode == kBPlain) y = f2bf(total);
        else if (kMode == kBResidual) y = bf_add(f2bf(total), res[o]);
        else y = bf_mul(f2bf(silu(rbf(total))), f2bf(total2));
        out[o] = y;
      }
    }
  }
}

// Embedding rows of tokens [first, first + m) of the call (prefill.embed,
// qwen35_prefill.hex:69-108); block 0 clears the argmax key when asked.
__global__ __launch_bounds__(kBlock) void k_bembed(const uint64_t* __restrict__ params, int first,
                                                    const uint16_t* __restrict__ table, int hidden,
                                                    uint16_t* __restrict__ h,
                                                    unsigned long long* __restrict__ best) {
  const uint64_t token = params[1 + first + blockIdx.x];
  const uint16_t* row = table + token * (uint64_t)hidden;
  uint16_t* dst = h + (size_t)blockIdx.x * hidden;
  for (int i = threadIdx.x; i < hidden; i += blockDim.x) dst[i] = row[i];
  if (blockIdx.x == 0 && threadIdx.x == 0 && best) *best = 0ull;
}

// RMSNorm of each row (qwen35.normalize with rows = sequence,
// qwen35.hex:912-977): one block per row, the decode norm's arithmetic.
__global__ __launch_bounds__(kBlock) void k_bnorm(const uint16_t* __restrict__ x,
                                                   const float* __restrict__ w, int cols, float eps,
                                                   uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) u32x4 bn_xs[];
  __shared__ float red[4];
  const uint16_t* xr = x + (size_t)blockIdx.x * cols;
  NormIn nin;
  norm_prefetch(nin, xr, w, cols);
  norm_finish(nin, bn_xs, xr, w, cols, eps, red);
  u32x4* o = reinterpret_cast<u32x4*>(out + (size_t)blockIdx.x * cols);
  for (int i = threadIdx.x; i < (cols >> 3); i += blockDim.x) o[i] = bn_xs[i];
}

// Four-tap convolution of every token of the chunk, then the per-head L2
// norm of the Q and K heads (batch.prepare, batch_prepare.hex:3-158): the tap
// at position p < `first` reads the cache history slot p % 3 (still holding
// the rows before this chunk), later taps read the chunk's own rows. Block
// (KD-channel chunk, token).
__global__ __launch_bounds__(kBlock) void k_bprepare(
    const uint16_t* __restrict__ qkv, const uint16_t* __restrict__ cache, int64_t conv_base,
    const uint64_t* __restrict__ params, int first, const float* __restrict__ conv_w, int qkv_size,
    int key_dim, int key_heads, uint16_t* __restrict__ conv_out, uint16_t* __restrict__ q_out,
    uint16_t* __restrict__ k_out) {
  __shared__ float squares[256];
  __shared__ float total;
  const int t = blockIdx.y;
  const int64_t begin = (int64_t)params[0] + first;  // position of the chunk's row 0
  const int64_t position = begin + t;
  const int chunk = blockIdx.x, tid = threadIdx.x;
  const int ch = chunk * key_dim + tid;
  const bool active = tid < key_dim && ch < qkv_size;
  const int key_size = key_heads * key_dim;
  float value = 0.0f;
  if (active) {
    float taps[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int64_t p = position - 3 + k;
      float input = 0.0f;
      if (p >= 0)
        input = p < begin ? bf2f(cache[conv_base + (p % 3) * qkv_size + ch])
                          : bf2f(qkv[(size_t)(p - begin) * qkv_size + ch]);
      taps[k] = input * conv_w[(size_t)ch * 4 + k];
    }
    const float tap3 = bf2f(qkv[(size_t)t * qkv_size + ch]) * conv_w[(size_t)ch * 4 + 3];
    const float sum = (taps[0] + taps[2]) + (taps[1] + tap3);
    const uint16_t result = f2bf(silu(rbf(sum)));
    conv_out[(size_t)t * qkv_size + ch] = result;
    value = bf2f(result);
  }
  if (chunk >= 2 * key_heads) return;  // value heads: convolution only
  if (tid < key_dim) squares[tid] = value * value;
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
    for (int i = 0; i < key_dim; ++i) s += squares[i];
    total = s;
  }
  __syncthreads();
  if (tid < key_dim) {
    const float norm = nsqrt(total + bitsf(0x358637bdu));
    uint16_t* dst = (chunk < key_heads ? q_out : k_out) + (size_t)t * key_size;
    dst[(chunk % key_heads) * key_dim + tid] = f2bf(value / norm);
  }
}

// History commit after the chunk's reads: the last min(m, 3) raw QKV rows
// into slots position % 3 (batch.history, batch_prepare.hex:209-292).
__global__ __launch_bounds__(kBlock) void k_bhistory(const uint16_t* __restrict__ qkv, int m,
                                                      uint16_t* __restrict__ cache,
                                                      int64_t conv_base,
                                                      const uint64_t* __restrict__ params,
                                                      int first, int qkv_size) {
  const int kept = m < 3 ? m : 3;
  const int64_t begin = (int64_t)params[0] + first;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < (int64_t)kept * qkv_size;
       i += (int64_t)gridDim.x * blockDim.x) {
    const int t = m - kept + (int)(i / qkv_size);
    const int ch = (int)(i % qkv_size);
    cache[conv_base + ((begin + t) % 3) * qkv_size + ch] = qkv[(size_t)t * qkv_size + ch];
  }
}

// DeltaNet scan over the chunk's tokens with the F32 state in registers
// (batch.scan, batch_scan.hex:1-200): per token exactly the single-step
// arithmetic of k_delta (32 lanes per value channel, lane l owns key elements
// l, l+32, ...; serial from 0.0, 32-wide halving tree), 8 channels of one
// head per block. Requires key_dim <= 256 and value_dim % 8 == 0.
//
// The serial chain reads only LDS: per stage of kScanTokens tokens the
// block first stages the head's k and q rows (lane-major, lane l's elements
// l + 32 j contiguous), its channels' values, and every token's decay and
// rate (computed in parallel: they do not depend on the state).
constexpr int kScanTokens = 64;

__host__ __device__ constexpr size_t bscan_lds_bytes(int key_dim) {
  return (size_t)kScanTokens * key_dim * 2 * 2 + (size_t)kScanTokens * (2 + 8) * 4;
}

template <int KJ>  // key elements per lane: key_dim / 32
__global__ __launch_bounds__(kBlock) void k_bscan(
    const uint16_t* __restrict__ conv, const uint16_t* __restrict__ q,
    const uint16_t* __restrict__ k, const uint16_t* __restrict__ alpha,
    const uint16_t* __restrict__ beta, const float* __restrict__ dt, const float* __restrict__ a,
    float* __restrict__ state, int m, int value_size, int value_dim, int value_heads, int key_dim,
    int key_heads, int qkv_size, float scale, uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) unsigned char scan_lds[];
  uint16_t* sk = reinterpret_cast<uint16_t*>(scan_lds);
  uint16_t* sq = sk + kScanTokens * key_dim;
  float* sdecay = reinterpret_cast<float*>(sq + kScanTokens * key_dim);
  float* srate = sdecay + kScanTokens;
  float* sval = srate + kScanTokens;  // [token][8]
  const int c0 = blockIdx.x * 8;
  const int ch = threadIdx.x >> 5;
  const int c = c0 + ch;
  const int lane = threadIdx.x & 31, half = (threadIdx.x >> 5) & 1;
  const bool valid = c < value_size;
  const int cc = valid ? c : 0;
  const int head = min(c0, value_size - 1) / value_dim;
  const int kbase = (head % key_heads) * key_dim;
  const int key_size = key_heads * key_dim;
  constexpr int kj = KJ;
  const float dth = dt[head], ah = a[head];
  float s[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) s[j] = state[(size_t)cc * key_dim + lane + 32 * j];
  for (int t0 = 0; t0 < m; t0 += kScanTokens) {
    const int ts = min(kScanTokens, m - t0);
    // stage: k and q rows lane-major, values, decay and rate
    const int quads = key_dim >> 3;
    for (int idx = threadIdx.x; idx < ts * quads; idx += blockDim.x) {
      const int tt = idx / quads, qd = idx - tt * quads;
      const size_t src = (size_t)(t0 + tt) * key_size + kbase + 8 * qd;
      const u32x4 kq4 = *reinterpret_cast<const u32x4*>(k + src);
      const u32x4 qq4 = *reinterpret_cast<const u32x4*>(q + src);
      const uint32_t kw[4] = {kq4.x, kq4.y, kq4.z, kq4.w}, qw[4] = {qq4.x, qq4.y, qq4.z, qq4.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 8 * qd + e;
        const int dst = tt * key_dim + (i & 31) * kj + (i >> 5);
        sk[dst] = (uint16_t)(kw[e >> 1] >> (16 * (e & 1)));
        sq[dst] = (uint16_t)(qw[e >> 1] >> (16 * (e & 1)));
      }
    }
    for (int idx = threadIdx.x; idx < ts * 8; idx += blockDim.x) {
      const int tt = idx >> 3, cv = min(c0 + (idx & 7), value_size - 1);
      sval[idx] = bf2f(conv[(size_t)(t0 + tt) * qkv_size + 2 * key_size + cv]);
    }
    if (threadIdx.x < ts) {
      const int t = t0 + threadIdx.x;
      const float time_step = softplus(bf2f(alpha[(size_t)t * value_heads + head]) + dth);
      sdecay[threadIdx.x] = hexp(rbf(time_step * ah));
      srate[threadIdx.x] = rbf(sigmoid(bf2f(beta[(size_t)t * value_heads + head])));
    }
    __syncthreads();
    for (int tt = 0; tt < ts; ++tt) {
      const uint16_t* kr = sk + tt * key_dim + lane * kj;
      const uint16_t* qr = sq + tt * key_dim + lane * kj;
      float kv[KJ], qv[KJ];
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        kv[j] = bf2f(kr[j]);
        qv[j] = bf2f(qr[j]);
      }
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) acc += s[j] * kv[j];
      acc = tree32_lanes(acc);
      const float t_lo = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 0));
      const float t_hi = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 32));
      const float total = half ? t_hi : t_lo;
      const float decay = sdecay[tt];
      const float delta = (sval[tt * 8 + ch] - total * decay) * srate[tt];
      float acc2 = 0.0f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        s[j] = s[j] * decay + kv[j] * delta;
        acc2 += s[j] * qv[j];
      }
      acc2 = tree32_lanes(acc2);
      if (lane == 0 && valid) out[(size_t)(t0 + tt) * value_size + c] = f2bf(acc2 * scale);
    }
    __syncthreads();
  }
  if (valid) {
#pragma unroll
    for (int j = 0; j < KJ; ++j) state[(size_t)c * key_dim + lane + 32 * j] = s[j];
  }
}

// RoPE tables [cos x R/2 | sin x R/2] for the chunk's positions
// (qwen3.rope-frequency + rope-sincos, batch_full_prepare.hex:63-70).
__global__ __launch_bounds__(kBlock) void k_brope(const uint64_t* __restrict__ params, int first,
                                                   const float* __restrict__ freq, int half,
                                                   float* __restrict__ rope) {
  const float position = (float)(uint32_t)((int64_t)params[0] + first + blockIdx.x);
  float* r = rope + (size_t)blockIdx.x * 2 * half;
  for (int i = threadIdx.x; i < half; i += blockDim.x) {
    float s, c;
    sincos_q(position * freq[i], &s, &c);
    r[i] = c;
    r[half + i] = s;
  }
}

// MoE router logits of every token (batch.moe.router, batch_moe.hex:45-135):
// the decode router's S32 over the normalised row with F32 weights, rows
// [0, E) routed and row E the shared-expert gate. Block (4 rows, token).
__global__ __launch_bounds__(kBlock) void k_brouter(const uint16_t* __restrict__ x, int cols,
                                                     const float* __restrict__ w,
                                                     const float* __restrict__ shared_w,
                                                     int experts, float* __restrict__ logits) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = experts + 1;
  const int row = blockIdx.x * 4 + wave;
  const int t = blockIdx.y;
  const int rc = min(row, rows - 1);
  const float* wr = rc < experts ? w + (size_t)rc * cols : shared_w;
  const uint16_t* xr = x + (size_t)t * cols;
  // physical lane l = 2r + h: reference lane r's low (h = 0) or high (h = 1)
  // accumulator over elements l + 64k
  float acc = 0.0f;
  for (int i = lane; i < cols; i += 64) acc += bf2f(xr[i]) * wr[i];
  float v = acc + lane_down<1>(acc);
  v += lane_down<32>(v);
  v += lane_down<16>(v);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  if (lane == 0 && row < rows) logits[(size_t)t * rows + row] = v;
}

// k_brouter's logits with each weight row read once per 16 tokens: wave w of
// block (row group, token group) keeps rows 16 rg + 2 w and + 1 in registers
// (lane l: elements l + 64 k), the group's 16 token rows are staged in LDS,
// and every (row, token) sum runs in k_brouter's order (each lane's chain
// over k, then the same tree), so the logits are bit-identical. cols a
// multiple of 64, at most 2048.
constexpr int kRouterTokens = 16;
constexpr int kRouterRows = 16;  // 2 per wave, 8 waves
template <int KJ>  // cols / 64
__global__ __launch_bounds__(512) void k_brouter_shared(const uint16_t* __restrict__ x, int n,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ shared_w, int experts,
                                                        float* __restrict__ logits) {
  constexpr int cols = 64 * KJ;
  __shared__ uint16_t xs[kRouterTokens][cols];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = experts + 1;
  const int t0 = blockIdx.y * kRouterTokens;
  const int tn = min(kRouterTokens, n - t0);
  float wv[2][KJ];
#pragma unroll
  for (int r = 0; r < 2; ++r) {
    const int rc = min(blockIdx.x * kRouterRows + 2 * wave + r, rows - 1);
    const float* wr = rc < experts ? w + (size_t)rc * cols : shared_w;
#pragma unroll
    for (int k = 0; k < KJ; ++k) wv[r][k] = wr[lane + 64 * k];
  }
  constexpr int pieces = cols / 8;
  for (int i = threadIdx.x; i < tn * pieces; i += blockDim.x) {
    const int t = i / pieces, p = i - t * pieces;
    reinterpret_cast<u32x4*>(&xs[t][0])[p] = ldq(x + (size_t)(t0 + t) * cols, p);
  }
  __syncthreads();
  for (int t = 0; t < tn; ++t) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float acc = 0.0f;
#pragma unroll
      for (int k = 0; k < KJ; ++k)
        acc += bf2f(xs[t][lane + 64 * k]) * wv[r][k];
      float v = acc + lane_down<1>(acc);
      v += lane_down<32>(v);
      v += lane_down<16>(v);
      v += lane_down<8>(v);
      v += lane_down<4>(v);
      v += lane_down<2>(v);
      const int row = blockIdx.x * kRouterRows + 2 * wave + r;
      if (lane == 0 && row < rows) logits[(size_t)(t0 + t) * rows + row] = v;
    }
  }
}

// Top-k of each token's routed logits by the reference's rank,
// rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)}, and the softmax
// weights p_j = exp(l_j - l_0) / den with den summed left to right
// (batch.moe.select, batch_moe.hex:136-317). One block per token. With
// last_ids, the last token's ids are also written there (the layer's slot of
// the session's exported top-k).
__global__ __launch_bounds__(kBlock) void k_bselect(const float* __restrict__ logits, int experts,
                                                     int top_k, int* __restrict__ ids,
                                                     float* __restrict__ probs, int* __restrict__ last_ids) {
  extern __shared__ float bs_lg[];
  __shared__ float chosen[64];
  const int t = blockIdx.x;
  const float* lt = logits + (size_t)t * (experts + 1);
  for (int e = threadIdx.x; e < experts; e += blockDim.x) bs_lg[e] = lt[e];
  // NaN logits can make ranks collide: the largest expert index of a shared
  // rank takes it (the restatement's ascending scatter; an LDS maximum) and
  // an unassigned rank k keeps expert k; without NaNs the ranks are a
  // permutation.
  __shared__ int won[64];
  if (threadIdx.x < top_k) won[threadIdx.x] = -1;
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    const float le = bs_lg[e];
    int rank = 0;
    for (int i = 0; i < experts; ++i) {
      const float o = bs_lg[i];
      rank += (o > le) ? 1 : ((i < e && !(le > o)) ? 1 : 0);
    }
    if (rank < top_k) atomicMax(&won[rank], e);
  }
  __syncthreads();
  if (threadIdx.x < top_k) {
    const int e = won[threadIdx.x] >= 0 ? won[threadIdx.x] : threadIdx.x;
    ids[(size_t)t * top_k + threadIdx.x] = e;
    chosen[threadIdx.x] = bs_lg[e];
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    const float ex = lane < top_k ? hexp(chosen[lane] - chosen[0]) : 0.0f;
    float den = 0.0f;
    for (int j = 0; j < top_k; ++j) den = den + __shfl(ex, j, 64);
    if (lane < top_k) probs[(size_t)t * top_k + lane] = ex / den;
  }
  if (last_ids && t == (int)gridDim.x - 1 && threadIdx.x < top_k)
    last_ids[threadIdx.x] = ids[(size_t)t * top_k + threadIdx.x];
}

// Expert gate/up of every token (batch.moe.gate, batch_moe.hex:339-411):
// dual B256 over the normalised row; routed rows r < K*I use expert
// ids[slot = r / I], row r % I, and give bf16(silu(g)*u*p_slot); shared rows
// give bf16(bf16(bf16(silu(g))*u)*sigmoid(l_E)), with g, u the bf16 totals.
// Block (4 rows, token). Requires hidden % 8 == 0.
__global__ __launch_bounds__(kBlock) void k_bmoe_gate(
    const uint16_t* __restrict__ x, int hidden, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ sgate,
    const uint16_t* __restrict__ sup, const int* __restrict__ ids, const float* __restrict__ probs,
    const float* __restrict__ logits, int experts, int top_k, int inter, int shared_inter,
    uint16_t* __restrict__ active) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.y;
  const int rows = top_k * inter + shared_inter;
  const int r = blockIdx.x * 4 + wave;
  if (r >= rows) return;  // wave-uniform
  const bool routed = r < top_k * inter;
  const int slot = routed ? r / inter : 0;
  const uint16_t *wg, *wu;
  if (routed) {
    const size_t wrow = (size_t)ids[(size_t)t * top_k + slot] * inter + r % inter;
    wg = gate + wrow * hidden;
    wu = up + wrow * hidden;
  } else {
    wg = sgate + (size_t)(r - top_k * inter) * hidden;
    wu = sup + (size_t)(r - top_k * inter) * hidden;
  }
  const u32x4* xq = reinterpret_cast<const u32x4*>(x + (size_t)t * hidden);
  const u32x4* gq = reinterpret_cast<const u32x4*>(wg);
  const u32x4* uq = reinterpret_cast<const u32x4*>(wu);
  float ag[4] = {0.0f, 0.0f, 0.0f, 0.0f}, au[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int qi = lane; qi < (hidden >> 3); qi += 64) {
    const u32x4 xv = xq[qi];
    b256_acc(ag, xv, gq[qi]);
    b256_acc(au, xv, uq[qi]);
  }
  const float both = b256_tree2(ag, au);
  const float g = lane_value(both, 31), u = lane_value(both, 63);
  if (lane == 0) {
    const float gb = rbf(g), ub = rbf(u);
    const float activated = silu(gb);
    float y;
    if (routed) {
      y = (activated * ub) * probs[(size_t)t * top_k + slot];
    } else {
      const float shared_prob = sigmoid(logits[(size_t)t * (experts + 1) + experts]);
      y = rbf(rbf(activated) * ub) * shared_prob;
    }
    active[(size_t)t * rows + r] = f2bf(y);
  }
}

// k_bmoe_gate with the weights read once per chunk: the (token, slot)
// assignments bucketed by expert (k_moe_bucket), block = kGRows rows of
// expert blockIdx.y, each wave kGRowsPerWave of them with their gate and up
// quads (lane + 64 j) held in registers, applied to the expert's tokens in
// turn (the next token's input quads in flight); the epilogues of up to 64
// tokens run at once, one per lane. kShared: the shared expert
// over tokens [16 blockIdx.y, +16). Per (token, row) the arithmetic is
// k_bmoe_gate's: the B256 lane order over the quads, the tree and the
// epilogue, so the results are the same bits.
constexpr int kGRowsPerWave = 1;
constexpr int kGRows = 4 * kGRowsPerWave;  // rows per block
constexpr int kGSharedTokens = 16;

template <int NQ, bool kShared>
__global__ __launch_bounds__(kBlock) void k_bmoe_gate_grouped(
    const uint16_t* __restrict__ x, int hidden, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, const int* __restrict__ eoff, const int* __restrict__ order,
    const float* __restrict__ probs, const float* __restrict__ logits, int experts, int top_k, int inter,
    int shared_inter, int n, uint16_t* __restrict__ active) {
  constexpr int RW = kGRowsPerWave;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int width = kShared ? shared_inter : inter;
  const int r0 = blockIdx.x * kGRows + RW * wave;
  if (r0 >= width) return;  // wave-uniform
  const int e = kShared ? 0 : blockIdx.y;
  const int begin = kShared ? kGSharedTokens * blockIdx.y : eoff[e];
  const int count = kShared ? min(kGSharedTokens, n - begin) : eoff[e + 1] - begin;
  if (count <= 0) return;
  const int quads = hidden >> 3;
  const int rows = top_k * inter + shared_inter;
  u32x4 gw[RW][NQ], uw[RW][NQ];
#pragma unroll
  for (int k = 0; k < RW; ++k) {
    const int r = min(r0 + k, width - 1);
    const size_t wrow = kShared ? (size_t)r : (size_t)e * inter + r;
    const u32x4* gq = reinterpret_cast<const u32x4*>(gate + wrow * hidden);
    const u32x4* uq = reinterpret_cast<const u32x4*>(up + wrow * hidden);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      gw[k][j] = gq[min(lane + 64 * j, quads - 1)];
      uw[k][j] = uq[min(lane + 64 * j, quads - 1)];
    }
  }
  auto token = [&](int i) { return kShared ? begin + i : order[begin + i] / top_k; };
  auto load = [&](u32x4 (&xv)[NQ], int i) {
    const u32x4* xq = reinterpret_cast<const u32x4*>(x + (size_t)token(min(i, count - 1)) * hidden);
#pragma unroll
    for (int j = 0; j < NQ; ++j) xv[j] = xq[min(lane + 64 * j, quads - 1)];
  };
  // the epilogues of up to 64 tokens at once: lane j keeps the totals of
  // token (i & ~63) + j and applies k_bmoe_gate's epilogue to it
  float pg[RW], pu[RW];
  auto finish = [&](int b, int m) {
    if (lane >= m) return;
    const int i = b + lane;
    const int a = kShared ? 0 : order[begin + i];
    const int t = kShared ? begin + i : a / top_k;
#pragma unroll
    for (int k = 0; k < RW; ++k) {
      const int r = r0 + k;
      if (r >= width) continue;
      const float gb = rbf(pg[k]), ub = rbf(pu[k]);
      const float activated = silu(gb);
      if (kShared) {
        const float shared_prob = sigmoid(logits[(size_t)t * (experts + 1) + experts]);
        active[(size_t)t * rows + top_k * inter + r] = f2bf(rbf(rbf(activated) * ub) * shared_prob);
      } else {
        const int slot = a - t * top_k;
        active[(size_t)t * rows + slot * inter + r] = f2bf((activated * ub) * probs[a]);
      }
    }
  };
  auto compute = [&](const u32x4 (&xv)[NQ], int i) {
#pragma unroll
    for (int k = 0; k < RW; ++k) {
      float ag[4] = {0.0f, 0.0f, 0.0f, 0.0f}, au[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < NQ; ++j)
        if (lane + 64 * j < quads) {
          b256_acc(ag, xv[j], gw[k][j]);
          b256_acc(au, xv[j], uw[k][j]);
        }
      const float both = b256_tree2(ag, au);
      const float g = lane_value(both, 31), u = lane_value(both, 63);
      if (lane == (i & 63)) {
        pg[k] = g;
        pu[k] = u;
      }
    }
    if ((i & 63) == 63 || i == count - 1) finish(i & ~63, (i & 63) + 1);  // wave-uniform
  };
  u32x4 xa[NQ], xb[NQ];
  load(xa, 0);
#pragma unroll 1
  for (int i = 0; i < count; i += 2) {
    load(xb, i + 1);
    compute(xa, i);
    if (i + 1 < count) {
      load(xa, i + 2);
      compute(xb, i + 1);
    }
  }
}

// Expert down of every token (batch.moe.down, batch_moe.hex:453-563): B256
// over the K*I/2 routed pairs (pair p from expert ids[p / (I/2)], channel
// p % (I/2)) with the shared pairs p < SI/2 accumulated in the same lanes,
// then bf16(bf16(routed + residual) (+) bf16(shared)). Block (4 rows,
// token), numbered so that the blocks of one 4-row group, all tokens, run on
// one XCD in sequence (block b runs on XCD b mod 8; XCD x takes the groups
// x, x + 8, ... in ascending order): the group's rows of every expert, 4 KB
// each, are read from HBM once into that XCD's L2 and shared by the tokens
// routed there, instead of each token streaming its experts' whole
// matrices. Grid: 8 * n * ceil(ceil(hidden / 4) / 8) blocks. Requires
// inter % 8 == 0, shared_inter % 8 == 0 and shared_inter <= top_k * inter.
inline int bmoe_down_grid(int hidden, int n) { return 8 * n * (((hidden + 3) / 4 + 7) / 8); }

__global__ __launch_bounds__(kBlock) void k_bmoe_down(
    const uint16_t* __restrict__ active, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ sdown, const int* __restrict__ ids,
    const uint16_t* __restrict__ res, int hidden, int top_k, int inter, int shared_inter, int n,
    uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int local = (int)(blockIdx.x >> 3);
  const int group = (int)(blockIdx.x & 7) + 8 * (local / n), t = local % n;
  const int o = group * 4 + wave;
  if (o >= hidden) return;  // wave-uniform
  const int rows = top_k * inter + shared_inter;
  const int aq = top_k * inter / 8, iq = inter / 8, sq = shared_inter / 8;
  const u32x4* xa = reinterpret_cast<const u32x4*>(active + (size_t)t * rows);
  const int* idt = ids + (size_t)t * top_k;
  const u32x4* sw = reinterpret_cast<const u32x4*>(sdown + (size_t)o * shared_inter);
  float ar[4] = {0.0f, 0.0f, 0.0f, 0.0f}, as[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int qi = lane; qi < aq; qi += 64) {
    const int slot = qi / iq, ch = qi % iq;
    const u32x4* wr =
        reinterpret_cast<const u32x4*>(down + ((size_t)idt[slot] * hidden + o) * inter);
    b256_acc(ar, xa[qi], wr[ch]);
    if (qi < sq) b256_acc(as, xa[aq + qi], sw[qi]);
  }
  const float both = b256_tree2(ar, as);
  const float routed = lane_value(both, 31), shared = lane_value(both, 63);
  if (lane == 0) {
    const size_t i = (size_t)t * hidden + o;
    out[i] = bf_add(f2bf(routed + bf2f(res[i])), f2bf(shared));
  }
}

// k_bmoe_down with each wave on kDRows consecutive output rows of one token:
// the token's activation quads are read once into registers and used for
// every row, each row's weight quads are read once. Block = (kDRows-row
// group, kDTokens tokens), wave w on token 4 by + w; blocks numbered as in
// k_bmoe_down, a group's blocks (all tokens) on one XCD in sequence. Per
// (token, row) the products, the lane chains over qi = lane, lane + 64, ...
// (routed and shared), the tree and the epilogue are k_bmoe_down's, so the
// results are the same bits. NQ: quads per lane, ceil(top_k * inter / 512)
// rounded up to a power of two.
constexpr int kDRows = 8;
constexpr int kDTokens = kBlock / 64;
inline int bmoe_down_rows_grid(int hidden, int n) {
  const int groups = (hidden + kDRows - 1) / kDRows, tiles = (n + kDTokens - 1) / kDTokens;
  return 8 * tiles * ((groups + 7) / 8);
}

template <int NQ>
__global__ __launch_bounds__(kBlock) void k_bmoe_down_rows(
    const uint16_t* __restrict__ active, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ sdown, const int* __restrict__ ids,
    const uint16_t* __restrict__ res, int hidden, int top_k, int inter, int shared_inter, int n,
    uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tiles = (n + kDTokens - 1) / kDTokens;
  const int local = (int)(blockIdx.x >> 3);
  const int group = (int)(blockIdx.x & 7) + 8 * (local / tiles);
  const int t = (local % tiles) * kDTokens + wave;
  const int o0 = group * kDRows;
  if (o0 >= hidden || t >= n) return;  // wave-uniform
  const int rows = top_k * inter + shared_inter;
  const int aq = top_k * inter / 8, iq = inter / 8, sq = shared_inter / 8;
  const u32x4* xa = reinterpret_cast<const u32x4*>(active + (size_t)t * rows);
  const int* idt = ids + (size_t)t * top_k;
  u32x4 xv[NQ], xs[NQ];
  size_t woff[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int qi = min(lane + 64 * j, aq - 1), slot = qi / iq, ch = qi - slot * iq;
    xv[j] = xa[qi];
    woff[j] = (size_t)idt[slot] * hidden * inter + (size_t)ch * 8;
    if (64 * j < sq) xs[j] = xa[aq + min(lane + 64 * j, sq - 1)];
  }
#pragma unroll
  for (int r = 0; r < kDRows; ++r) {
    const int o = o0 + r;
    if (o >= hidden) break;  // wave-uniform
    u32x4 wv[NQ], ws[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      wv[j] = *reinterpret_cast<const u32x4*>(down + woff[j] + (size_t)o * inter);
      if (64 * j < sq)
        ws[j] = reinterpret_cast<const u32x4*>(sdown + (size_t)o * shared_inter)[min(lane + 64 * j, sq - 1)];
    }
    float ar[4] = {0.0f, 0.0f, 0.0f, 0.0f}, as[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      if (lane + 64 * j < aq) b256_acc(ar, xv[j], wv[j]);
      if (lane + 64 * j < sq) b256_acc(as, xs[j], ws[j]);
    }
    const float both = b256_tree2(ar, as);
    const float routed = lane_value(both, 31), shared = lane_value(both, 63);
    if (lane == 0) {
      const size_t i = (size_t)t * hidden + o;
      out[i] = bf_add(f2bf(routed + bf2f(res[i])), f2bf(shared));
    }
  }
}

}  // namespace cq35
