// Weight-shared decode step for independent sessions (same model and
// capacity, one token each): every layer's weights are read once for all the
// sessions' tokens instead of once per session.
//
// The reference steps sessions one after another (src/server/engine.rs:
// 143-207); each token's arithmetic here is exactly its single-session
// decode step: the GEMVs below keep every token's split-pair lane order and
// halving tree (S32 / S64 / S256, the per-token kernels of gemv.h), only the
// weight quads are loaded once and applied to NB tokens held in LDS. The
// per-token kernels of layers.h (convolution, delta rule, gated norm, full
// prepare, staged attention) run with one grid row per session and a
// SessionRows table of cache pointers and positions.
//
// Block mapping. A GEMV grid is (row blocks) x (token groups of NB). Blocks
// are dealt to the 8 XCDs round-robin, so the token groups that share a row
// block are placed on one XCD (block b: XCD b mod 8): the first reads the
// weights from HBM and the others from that XCD's L2.
#pragma once

#include "layers.h"

namespace cq35 {

constexpr int kBatchNB = 4;      // tokens per S32 GEMV block (S64 launches use 2)
constexpr int kBatchNBDual = 2;  // tokens per dual S256 (SwiGLU) block
constexpr int kBatchChunk = 2048;  // input columns staged per pass

// (row block, token group) of block b for `groups` token groups.
__device__ __forceinline__ void batch_block(int b, int groups, int* rb, int* tg) {
  const int x = b & 7, r = b >> 3;
  *tg = r % groups;
  *rb = (r / groups) * 8 + x;
}
inline int batch_grid(int row_blocks, int groups) {
  return ((row_blocks + 7) / 8) * 8 * groups;
}

// Stage columns k0 .. k0 + ch of rows t0 .. t0 + NB of x [tokens][cols] into
// LDS as F32 (rows past `tokens` are zero and never stored), so the
// accumulation loops read their inputs already widened. Row t takes ch
// floats: quad o's elements 0-3 at [4o, 4o + 4) of its first half and 4-7 at
// the same place in its second half, so lanes reading consecutive quads read
// 16-byte-consecutive words (no bank conflicts).
template <int NB>
__device__ __forceinline__ void stage_f32(float* xf, const uint16_t* __restrict__ x, int tokens, int t0, int cols,
                                          int k0, int ch) {
  const int n8 = ch >> 3;
  __syncthreads();  // the previous chunk's readers are done
  for (int i = threadIdx.x; i < NB * n8; i += blockDim.x) {
    const int t = i / n8, o = i - t * n8;
    const u32x4 v = t0 + t < tokens ? ldq(x + (size_t)(t0 + t) * cols + k0, o) : u32x4{0u, 0u, 0u, 0u};
    f32x4* row = reinterpret_cast<f32x4*>(xf + (size_t)t * ch);
    row[o] = f32x4{lo2f(v.x), hi2f(v.x), lo2f(v.y), hi2f(v.y)};
    row[n8 + o] = f32x4{lo2f(v.z), hi2f(v.z), lo2f(v.w), hi2f(v.w)};
  }
  __syncthreads();
}

// acc += the four pairs of quad o of a staged row of `n8` quads times weight
// quad w: quad_acc's products and sums, in its order.
__device__ __forceinline__ void quad_acc_staged(Quad& a, const float* xrow, int n8, int o, const u32x4& w) {
  const f32x4 p = reinterpret_cast<const f32x4*>(xrow)[o];
  const f32x4 r = reinterpret_cast<const f32x4*>(xrow)[n8 + o];
  const float xl[4] = {p.x, p.z, r.x, r.z}, xh[4] = {p.y, p.w, r.y, r.w};
  quad_acc_f(a, xl, xh, w);
}

// Embedding rows and per-session RoPE tables (k_embed for every session):
// grid (blocks over hidden, sessions); block 0 of a row also clears the
// session's argmax key.
__global__ __launch_bounds__(kBlock) void k_sembed(const SessionRows* __restrict__ rows,
                                                    const uint16_t* __restrict__ table, int hidden,
                                                    uint16_t* __restrict__ h, const float* __restrict__ freq,
                                                    int half, float* __restrict__ rope,
                                                    unsigned long long* __restrict__ best) {
  const int y = blockIdx.y;
  const uint64_t token = rows->token[y];
  const uint16_t* row = table + token * (uint64_t)hidden;
  uint16_t* hy = h + (size_t)y * hidden;
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < hidden; i += gridDim.x * blockDim.x) hy[i] = row[i];
  if (blockIdx.x == 0) {
    const float position = (float)(uint32_t)rows->position[y];
    float* ry = rope + (size_t)y * 2 * half;
    for (int i = threadIdx.x; i < half; i += blockDim.x) {
      float s, c;
      sincos_q(position * freq[i], &s, &c);
      ry[i] = c;
      ry[half + i] = s;
    }
    if (threadIdx.x == 0) best[y] = 0ull;
  }
}

// S32 over rows of up to four segments (k_project32's order: 8 lanes per
// row, lane q holding reference lanes 4q..4q+3, visiting its quads q, q + 8,
// ... in order, the staged column chunks in order) for NB tokens of already
// normalised rows; token t's output row r of segment s goes to
// seg.out[s][t * seg.rows[s] + r]. kArgmax: the vocabulary head, with each
// token's (value, lowest index) maximum into best[t].
template <bool kArgmax, int kNQ, int NB = kBatchNB>
__global__ __launch_bounds__(kBlock) void k_ws32(const uint16_t* __restrict__ x, int tokens, int groups,
                                                 Segments seg, int cols, unsigned long long* __restrict__ best) {
  constexpr int NQ = kNQ;
  extern __shared__ __align__(16) float xf[];  // [NB][chunk]
  __shared__ unsigned long long wave_best[4][NB];
  int rb, tg;
  batch_block(blockIdx.x, groups, &rb, &tg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 7, g = lane >> 3;
  const int total = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int row = (rb * 4 + wave) * 8 + g;
  const int t0 = tg * NB;
  int local;
  const int s = segment_of(seg, min(row, total - 1), &local);
  const uint16_t* wr = segment_w(seg, s) + (size_t)local * cols;
  const int srows = s == 0 ? seg.rows[0] : s == 1 ? seg.rows[1] : s == 2 ? seg.rows[2] : seg.rows[3];
  Quad acc[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) quad_zero(acc[t]);
  for (int k0 = 0; k0 < cols; k0 += kBatchChunk) {
    const int ch = min(kBatchChunk, cols - k0), cq = ch >> 3, qb = k0 >> 3;
    u32x4 wv[NQ];
#pragma unroll
    for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, qb + min(q + 8 * j, cq - 1));
    stage_f32<NB>(xf, x, tokens, t0, cols, k0, ch);
    for (int b = 0; b * 8 * NQ < cq; ++b) {
      if (b > 0) {
#pragma unroll
        for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, qb + min(q + 8 * (NQ * b + j), cq - 1));
      }
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int o = q + 8 * (NQ * b + j);
        if (o < cq) {
#pragma unroll
          for (int t = 0; t < NB; ++t) quad_acc_staged(acc[t], xf + t * ch, cq, o, wv[j]);
        }
      }
    }
  }
  unsigned long long mine[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const float v = quad_tree<8>(acc[t]);
    mine[t] = 0ull;
    if (q == 0 && row < total && t0 + t < tokens) {
      const uint16_t bb = f2bf(v);
      segment_out(seg, s)[(size_t)(t0 + t) * srows + local] = bb;
      if (kArgmax) mine[t] = logit_key(bb, (uint32_t)row);
    }
  }
  if (kArgmax) {
#pragma unroll
    for (int t = 0; t < NB; ++t) {
#pragma unroll
      for (int d = 32; d >= 8; d >>= 1) {
        const unsigned long long o = __shfl_down(mine[t], d, 64);
        mine[t] = o > mine[t] ? o : mine[t];
      }
      if (lane == 0) wave_best[wave][t] = mine[t];
    }
    __syncthreads();
    if (threadIdx.x < NB && t0 + (int)threadIdx.x < tokens) {
      const int t = threadIdx.x;
      unsigned long long bv = wave_best[0][t];
#pragma unroll
      for (int i = 1; i < 4; ++i) bv = wave_best[i][t] > bv ? wave_best[i][t] : bv;
      if (bv) atomicMax(best + t0 + t, bv);
    }
  }
}

// S64 + residual (k_residual's order: 16 lanes per row, lane q visiting its
// quads q, q + 16, ... in order) for NB tokens:
// out[t][r] = bf16(bf16(tree64(x_t . w_r)) (+) res[t][r]). Four waves of four
// rows per block; the input staged in column chunks.
template <int kNQ, int NB = kBatchNB>
__global__ __launch_bounds__(kBlock) void k_ws64(const uint16_t* __restrict__ x, int tokens, int groups,
                                                 const uint16_t* __restrict__ w, int rows, int cols,
                                                 const uint16_t* __restrict__ res, uint16_t* __restrict__ out) {
  constexpr int NQ = kNQ;
  extern __shared__ __align__(16) float xf[];  // [NB][chunk]
  int rb, tg;
  batch_block(blockIdx.x, groups, &rb, &tg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, q = lane & 15, g = lane >> 4;
  const int row = (rb * 4 + wave) * 4 + g;
  const int t0 = tg * NB;
  const uint16_t* wr = w + (size_t)min(row, rows - 1) * cols;
  Quad acc[NB];
#pragma unroll
  for (int t = 0; t < NB; ++t) quad_zero(acc[t]);
  for (int k0 = 0; k0 < cols; k0 += kBatchChunk) {
    const int ch = min(kBatchChunk, cols - k0), cq = ch >> 3, qb = k0 >> 3;
    u32x4 wv[NQ];
    if (cq % (16 * NQ) == 0) {
      // whole batches (every shipped width): no clamps or per-quad guards,
      // the same quads in the same order
      const u32x4* wq = reinterpret_cast<const u32x4*>(wr) + qb + q;
#pragma unroll
      for (int j = 0; j < NQ; ++j) wv[j] = wq[16 * j];
      stage_f32<NB>(xf, x, tokens, t0, cols, k0, ch);
      for (int b = 0; b * 16 * NQ < cq; ++b) {
        if (b > 0) {
#pragma unroll
          for (int j = 0; j < NQ; ++j) wv[j] = wq[16 * (NQ * b + j)];
        }
#pragma unroll
        for (int j = 0; j < NQ; ++j) {
          const int o = q + 16 * (NQ * b + j);
#pragma unroll
          for (int t = 0; t < NB; ++t) quad_acc_staged(acc[t], xf + t * ch, cq, o, wv[j]);
        }
      }
      continue;
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, qb + min(q + 16 * j, cq - 1));
    stage_f32<NB>(xf, x, tokens, t0, cols, k0, ch);
    for (int b = 0; b * 16 * NQ < cq; ++b) {
      if (b > 0) {
#pragma unroll
        for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, qb + min(q + 16 * (NQ * b + j), cq - 1));
      }
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int o = q + 16 * (NQ * b + j);
        if (o < cq) {
#pragma unroll
          for (int t = 0; t < NB; ++t) quad_acc_staged(acc[t], xf + t * ch, cq, o, wv[j]);
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NB; ++t) {
    const float v = quad_tree<16>(acc[t]);
    if (q == 0 && row < rows && t0 + t < tokens) {
      const size_t o = (size_t)(t0 + t) * rows + row;
      out[o] = res ? bf_add(f2bf(v), res[o]) : f2bf(v);
    }
  }
}

// Dense SwiGLU gate/up (k_gate_up<false>'s dual S256 order: lane l visiting
// quads l, l + 64, ... in order, kRowsGate rows per wave) for NB tokens of
// already normalised rows: act[t][r] = bf16(bf16(silu(bf16 g)) * bf16(u)).
// The input is staged once (cols <= kBatchChunk).
template <int NB = kBatchNBDual>
__global__ __launch_bounds__(kBlock) void k_ws256_swiglu(const uint16_t* __restrict__ x, int tokens, int groups,
                                                         const uint16_t* __restrict__ gate,
                                                         const uint16_t* __restrict__ up, int rows, int cols,
                                                         uint16_t* __restrict__ act) {
  constexpr int RW = kRowsGate, NQ = 4;
  extern __shared__ __align__(16) float xf[];  // [NB][cols]
  int rb, tg;
  batch_block(blockIdx.x, groups, &rb, &tg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quads = cols >> 3;
  const int row0 = (rb * 4 + wave) * RW;
  const int t0 = tg * NB;
  u32x4 gv[RW][NQ], uv[RW][NQ];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const int row = min(row0 + r, rows - 1);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      gv[r][j] = ldq(gate + (size_t)row * cols, min(lane + 64 * j, quads - 1));
      uv[r][j] = ldq(up + (size_t)row * cols, min(lane + 64 * j, quads - 1));
    }
  }
  stage_f32<NB>(xf, x, tokens, t0, cols, 0, cols);
  // each (row, token) total pair, wave-uniform; the epilogues run afterwards
  // one per lane (item i = r * NB + t on lane i) instead of once per item
  constexpr int NI = RW * NB;
  static_assert(NI <= 64, "epilogue lanes");
  float gs[NI], us[NI];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    Quad ga[NB], ua[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      quad_zero(ga[t]);
      quad_zero(ua[t]);
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (lane + 64 * j < quads) {
#pragma unroll
        for (int t = 0; t < NB; ++t) {
          quad_acc_staged(ga[t], xf + t * cols, quads, lane + 64 * j, gv[r][j]);
          quad_acc_staged(ua[t], xf + t * cols, quads, lane + 64 * j, uv[r][j]);
        }
      }
#pragma unroll
    for (int t = 0; t < NB; ++t) {
      const float tot = quad_tree64_pair_end(ga[t], ua[t]);  // gate total in lane 31, up total in lane 63
      gs[r * NB + t] = lane_value(tot, 31);
      us[r * NB + t] = lane_value(tot, 63);
    }
  }
  float gsum = 0.0f, usum = 0.0f;
#pragma unroll
  for (int i = 0; i < NI; ++i)
    if (lane == i) {
      gsum = gs[i];
      usum = us[i];
    }
  const int r = lane / NB, t = lane - (lane / NB) * NB;
  const int row = row0 + r;
  if (lane < NI && row < rows && t0 + t < tokens)
    act[(size_t)(t0 + t) * rows + row] = bf_mul(f2bf(silu(rbf(gsum))), f2bf(usum));
}

}  // namespace cq35
