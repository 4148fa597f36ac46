// Batch-1 BF16 GEMV family for gfx950 with the reference's exact reduction.
//
// The reference accumulates a row as W "reference lanes": lane r visits the
// BF16 pairs r, r+W, r+2W, ... in order, keeping separate low/high F32
// accumulators, and the W lane values (low + high) are combined by a halving
// tree (tests/qwen35_simt.rs:99-116; qwen35_simt.hex:4-120, 240-346). W is 32
// (project, router, MoE down), 64 (residual) or 256 (grouped projections,
// SwiGLU, MoE gate/up).
//
// Mapping onto wave64 with 128-bit loads: a physical lane q owns reference
// lanes 4q..4q+3, so one 16-byte load per chunk hands it exactly the four
// pairs those lanes read in that chunk, and the per-lane order is preserved.
// A row therefore occupies LPR = W/4 physical lanes (8, 16 or 64) and a wave
// streams 64/LPR rows at once. The tree runs with cross-lane shuffles for
// reference strides >= 4 and finishes inside the lane (strides 2, 1).
//
// Requires pairs % 4 == 0 (hidden, expert and head widths are multiples of
// 8 elements in every Qwen3.5/3.6 shape; validated on the host).
#pragma once

#include "numerics.h"

namespace cq35 {

constexpr int kBlock = 256;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

struct Quad {
  float lo[4];
  float hi[4];
};

__device__ __forceinline__ void quad_zero(Quad& a) {
#pragma unroll
  for (int k = 0; k < 4; ++k) a.lo[k] = a.hi[k] = 0.0f;
}

// acc.lo += x.lo * w.lo; acc.hi += x.hi * w.hi for four pairs, each product
// and sum rounded separately (dot-pair order of qwen35_simt.hex:40-45).
__device__ __forceinline__ void quad_acc(Quad& a, const u32x4& x, const u32x4& w) {
  a.lo[0] += lo2f(x.x) * lo2f(w.x); a.hi[0] += hi2f(x.x) * hi2f(w.x);
  a.lo[1] += lo2f(x.y) * lo2f(w.y); a.hi[1] += hi2f(x.y) * hi2f(w.y);
  a.lo[2] += lo2f(x.z) * lo2f(w.z); a.hi[2] += hi2f(x.z) * hi2f(w.z);
  a.lo[3] += lo2f(x.w) * lo2f(w.w); a.hi[3] += hi2f(x.w) * hi2f(w.w);
}

// F32 weights (the MoE router, qwen35_simt.hex:122-239): a quad of pairs is
// eight floats.
__device__ __forceinline__ void quad_acc_f32(Quad& a, const u32x4& x, const f32x4& w0,
                                             const f32x4& w1) {
  a.lo[0] += lo2f(x.x) * w0.x; a.hi[0] += hi2f(x.x) * w0.y;
  a.lo[1] += lo2f(x.y) * w0.z; a.hi[1] += hi2f(x.y) * w0.w;
  a.lo[2] += lo2f(x.z) * w1.x; a.hi[2] += hi2f(x.z) * w1.y;
  a.lo[3] += lo2f(x.w) * w1.z; a.hi[3] += hi2f(x.w) * w1.w;
}

// Halving tree of width W = 4*LPR over the reference lanes held by the LPR
// physical lanes of a row group. Must be reached by every lane of the wave.
// The result is valid in the group's first lane.
template <int LPR>
__device__ __forceinline__ float quad_tree(const Quad& a) {
  float v0 = a.lo[0] + a.hi[0];
  float v1 = a.lo[1] + a.hi[1];
  float v2 = a.lo[2] + a.hi[2];
  float v3 = a.lo[3] + a.hi[3];
#pragma unroll
  for (int s = LPR / 2; s >= 1; s >>= 1) {
    v0 += __shfl_down(v0, s, 64);
    v1 += __shfl_down(v1, s, 64);
    v2 += __shfl_down(v2, s, 64);
    v3 += __shfl_down(v3, s, 64);
  }
  v0 += v2;
  v1 += v3;
  return v0 + v1;
}

// Copy a BF16 vector of `pairs` pairs into LDS (as packed u32 pairs).
__device__ __forceinline__ void stage_pairs(uint32_t* lds, const uint16_t* x, int pairs) {
  const u32x4* src = reinterpret_cast<const u32x4*>(x);
  u32x4* dst = reinterpret_cast<u32x4*>(lds);
  for (int i = threadIdx.x; i < pairs / 4; i += blockDim.x) dst[i] = src[i];
  __syncthreads();
}

// Accumulate one row against the staged input: physical lane q reads quads
// j*LPR + q (pairs 4(j*LPR+q) .. +3 = chunk j, reference lanes 4q..4q+3).
template <int LPR>
__device__ __forceinline__ void row_accumulate(Quad& acc, const uint32_t* xs, const uint16_t* wrow,
                                               int pairs, int q) {
  const u32x4* w4 = reinterpret_cast<const u32x4*>(wrow);
  const u32x4* x4 = reinterpret_cast<const u32x4*>(xs);
  const int quads = pairs >> 2;
#pragma unroll 8
  for (int i = q; i < quads; i += LPR) quad_acc(acc, x4[i], w4[i]);
}

// ---------------------------------------------------------------- kernels

// Up to four row-major matrices sharing one input (group-project,
// group_projection.hex:3-97, and the consecutive fused.project launches of
// the dense graph). Rows are numbered across segments.
struct Segments {
  const uint16_t* w[4];
  uint16_t* out[4];
  int rows[4];
  int count;
};

enum Epilogue { kStoreBf16 = 0, kResidual = 1 };

template <int W, int EPI>
__global__ __launch_bounds__(kBlock) void k_project(const uint16_t* __restrict__ x, Segments seg,
                                                     int pairs, const uint16_t* __restrict__ res) {
  constexpr int LPR = W / 4, RPW = 64 / LPR, RPB = 4 * RPW;
  extern __shared__ __align__(16) uint32_t xs[];
  stage_pairs(xs, x, pairs);
  const int total = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane % LPR, g = lane / LPR;
  for (int base = blockIdx.x * RPB; base < total; base += gridDim.x * RPB) {
    const int row = base + wave * RPW + g;
    int s = 0, local = row;
    while (s < 3 && local >= seg.rows[s]) { local -= seg.rows[s]; ++s; }
    Quad acc;
    quad_zero(acc);
    if (row < total) row_accumulate<LPR>(acc, xs, seg.w[s] + (size_t)local * (2 * pairs), pairs, q);
    const float v = quad_tree<LPR>(acc);
    if (q == 0 && row < total) {
      if (EPI == kResidual)
        seg.out[s][local] = bf_add(f2bf(v), res[local]);  // simt.hex:442-454
      else
        seg.out[s][local] = f2bf(v);                      // simt.hex:400-410
    }
  }
}

// Orderable key of a BF16 logit for a (value, first index) maximum: larger
// value wins, equal values prefer the lower index; -0 equals +0; NaN never
// wins. key 0 means "no candidate" (fused_argmax.hex:1-104 semantics).
__device__ __forceinline__ unsigned long long logit_key(uint16_t b, uint32_t index) {
  float v = bf2f(b);
  if (v != v) return 0ull;
  uint32_t u = v == 0.0f ? 0u : fbits(v);
  uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ordered << 32) | (unsigned long long)(0xffffffffu - index);
}

// Vocabulary head: S32 projection to BF16 logits fused with the greedy
// argmax (simt.hex:348-441 + fused_argmax.hex), reduced through one 64-bit
// atomic max per block.
__global__ __launch_bounds__(kBlock) void k_logits(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ w, int rows,
                                                    int pairs, uint16_t* __restrict__ logits,
                                                    unsigned long long* __restrict__ best) {
  constexpr int LPR = 8, RPW = 8, RPB = 32;
  extern __shared__ __align__(16) uint32_t xs[];
  __shared__ unsigned long long wave_best[kBlock / 64];
  stage_pairs(xs, x, pairs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane % LPR, g = lane / LPR;
  unsigned long long mine = 0ull;
  for (int base = blockIdx.x * RPB; base < rows; base += gridDim.x * RPB) {
    const int row = base + wave * RPW + g;
    Quad acc;
    quad_zero(acc);
    if (row < rows) row_accumulate<LPR>(acc, xs, w + (size_t)row * (2 * pairs), pairs, q);
    const float v = quad_tree<LPR>(acc);
    if (q == 0 && row < rows) {
      const uint16_t b = f2bf(v);
      logits[row] = b;
      const unsigned long long k = logit_key(b, (uint32_t)row);
      mine = k > mine ? k : mine;
    }
  }
  for (int s = 32; s >= 1; s >>= 1) {
    const unsigned long long o = __shfl_down(mine, s, 64);
    mine = o > mine ? o : mine;
  }
  if (lane == 0) wave_best[wave] = mine;
  __syncthreads();
  if (threadIdx.x == 0) {
    unsigned long long b = wave_best[0];
    for (int i = 1; i < kBlock / 64; ++i) b = wave_best[i] > b ? wave_best[i] : b;
    if (b) atomicMax(best, b);
  }
}

// MoE router: S32 over BF16 input x F32 weights, E routed rows then the
// shared-expert gate row, F32 logits (moe.hex:4-84).
__global__ __launch_bounds__(kBlock) void k_router(const uint16_t* __restrict__ x,
                                                    const float* __restrict__ w,
                                                    const float* __restrict__ shared_w, int experts,
                                                    int pairs, float* __restrict__ logits) {
  constexpr int LPR = 8, RPW = 8, RPB = 32;
  extern __shared__ __align__(16) uint32_t xs[];
  stage_pairs(xs, x, pairs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane % LPR, g = lane / LPR;
  const int rows = experts + 1;
  for (int base = blockIdx.x * RPB; base < rows; base += gridDim.x * RPB) {
    const int row = base + wave * RPW + g;
    Quad acc;
    quad_zero(acc);
    if (row < rows) {
      const float* wr = row < experts ? w + (size_t)row * (2 * pairs) : shared_w;
      const f32x4* w4 = reinterpret_cast<const f32x4*>(wr);
      const u32x4* x4 = reinterpret_cast<const u32x4*>(xs);
      for (int i = q; i < pairs / 4; i += LPR) quad_acc_f32(acc, x4[i], w4[2 * i], w4[2 * i + 1]);
    }
    const float v = quad_tree<LPR>(acc);
    if (q == 0 && row < rows) logits[row] = v;
  }
}

// Dense SwiGLU: dual S256 over gate and up rows, bf16(silu(bf16 g)) (x)
// bf16(u) (qwen3.fused.gate, simt.hex:539-646).
__global__ __launch_bounds__(kBlock) void k_swiglu(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ wg,
                                                    const uint16_t* __restrict__ wu, int rows,
                                                    int pairs, uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) uint32_t xs[];
  stage_pairs(xs, x, pairs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
    Quad g, u;
    quad_zero(g);
    quad_zero(u);
    if (row < rows) {
      row_accumulate<64>(g, xs, wg + (size_t)row * (2 * pairs), pairs, lane);
      row_accumulate<64>(u, xs, wu + (size_t)row * (2 * pairs), pairs, lane);
    }
    const float gv = quad_tree<64>(g);
    const float uv = quad_tree<64>(u);
    if (lane == 0 && row < rows) out[row] = bf_mul(f2bf(silu(rbf(gv))), f2bf(uv));
  }
}

// Routed + shared expert gate/up (moe.hex:254-333): rows [0, K*I) belong to
// the selected experts in rank order, rows [K*I, K*I+SI) to the shared
// expert. Routed: bf16(silu(g) * u * p_slot); shared:
// bf16(bf16(bf16(silu(g)) * u) * sigmoid(shared logit)).
__global__ __launch_bounds__(kBlock) void k_moe_gate(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ sgate,
    const uint16_t* __restrict__ sup, const int* __restrict__ ids, const float* __restrict__ probs,
    const float* __restrict__ router, int experts, int top_k, int inter, int shared_inter,
    int pairs, uint16_t* __restrict__ active) {
  extern __shared__ __align__(16) uint32_t xs[];
  stage_pairs(xs, x, pairs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int routed_rows = top_k * inter, rows = routed_rows + shared_inter;
  const float shared_prob = sigmoid(router[experts]);
  for (int row = blockIdx.x * 4 + wave; row < rows; row += gridDim.x * 4) {
    Quad g, u;
    quad_zero(g);
    quad_zero(u);
    const bool routed = row < routed_rows;
    int slot = 0;
    if (row < rows) {
      const uint16_t *wg, *wu;
      if (routed) {
        slot = row / inter;
        const size_t r = (size_t)ids[slot] * inter + (row % inter);
        wg = gate + r * (2 * pairs);
        wu = up + r * (2 * pairs);
      } else {
        wg = sgate + (size_t)(row - routed_rows) * (2 * pairs);
        wu = sup + (size_t)(row - routed_rows) * (2 * pairs);
      }
      row_accumulate<64>(g, xs, wg, pairs, lane);
      row_accumulate<64>(u, xs, wu, pairs, lane);
    }
    const float gv = quad_tree<64>(g);
    const float uv = quad_tree<64>(u);
    if (lane == 0 && row < rows) {
      const float gb = rbf(gv), ub = rbf(uv);
      const float activated = silu(gb);
      float y;
      if (routed) y = (activated * ub) * probs[slot];
      else y = rbf(rbf(activated) * ub) * shared_prob;
      active[row] = f2bf(y);
    }
  }
}

// Expert down projection (moe.hex:371-434, simt_moe.hex:36-287): per hidden
// row, S32 over the concatenated routed activations (pair p reads expert
// ids[p / (I/2)]) and a separate S32 over the shared activations;
// out = bf16(bf16(routed + residual) (+) bf16(shared)).
__global__ __launch_bounds__(kBlock) void k_moe_down(
    const uint16_t* __restrict__ active, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ sdown, const int* __restrict__ ids,
    const uint16_t* __restrict__ residual, int hidden, int top_k, int inter, int shared_inter,
    uint16_t* __restrict__ out) {
  constexpr int LPR = 8, RPW = 8, RPB = 32;
  extern __shared__ __align__(16) uint32_t xs[];
  const int routed_pairs = top_k * inter / 2, shared_pairs = shared_inter / 2;
  stage_pairs(xs, active, routed_pairs + shared_pairs);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane % LPR, g = lane / LPR;
  const int ip = inter / 2;
  const u32x4* x4 = reinterpret_cast<const u32x4*>(xs);
  for (int base = blockIdx.x * RPB; base < hidden; base += gridDim.x * RPB) {
    const int row = base + wave * RPW + g;
    Quad r, s;
    quad_zero(r);
    quad_zero(s);
    if (row < hidden) {
#pragma unroll 4
      for (int i = q; i < routed_pairs / 4; i += LPR) {
        const int p = 4 * i;
        const int slot = p / ip;
        const u32x4* w4 = reinterpret_cast<const u32x4*>(
            down + ((size_t)ids[slot] * hidden + row) * inter + 2 * (p - slot * ip));
        quad_acc(r, x4[i], *w4);
      }
      const u32x4* s4 = reinterpret_cast<const u32x4*>(sdown + (size_t)row * shared_inter);
      const u32x4* xs4 = x4 + routed_pairs / 4;
#pragma unroll 4
      for (int i = q; i < shared_pairs / 4; i += LPR)
        quad_acc(s, xs4[i], s4[i]);
    }
    const float rv = quad_tree<LPR>(r);
    const float sv = quad_tree<LPR>(s);
    if (q == 0 && row < hidden) {
      const uint16_t routed_bf = f2bf(rv + bf2f(residual[row]));
      out[row] = bf_add(routed_bf, f2bf(sv));
    }
  }
}

}  // namespace cq35
