// Batch-1 BF16 GEMV family for gfx950 with the reference's exact reduction.
//
// The reference accumulates a row as W "reference lanes": lane r visits the
// BF16 pairs r, r+W, r+2W, ... in order, keeping separate low/high F32
// accumulators, and the W lane values (low + high) are combined by a halving
// tree (tests/qwen35_simt.rs:99-116; qwen35_simt.hex:4-120, 240-346). W is 32
// (project, router, MoE down, vocabulary head), 64 (residual) or 256
// (grouped projections, SwiGLU, MoE gate/up).
//
// Mapping onto wave64 with 128-bit loads: a physical lane q owns reference
// lanes 4q..4q+3, so one 16-byte load ("quad", four pairs) hands it exactly
// the four pairs those lanes read in that chunk, and the per-lane order is
// preserved. A row occupies LPR = W/4 physical lanes (8, 16 or 64). The tree
// runs with cross-lane shuffles for reference strides >= 4 and finishes
// inside the lane (strides 2, 1).
//
// Memory-level parallelism is the whole game at batch 1. Every kernel
//  1. issues the loads of its input row (and norm weights) first,
//  2. then all the weight loads of its tile into a statically indexed
//     register array (clamped addresses, no branches between the loads),
//  3. and only then waits, for the input alone (the vector-memory counter
//     retires in order), stages it in LDS and consumes the weights,
// so each lane keeps 16-32 loads in flight instead of one.
//
// Inputs that the reference normalises first (qwen35.normalize before every
// projection) are normalised inside the consuming kernel: each block
// recomputes the RMS norm of the hidden row while its weight loads are in
// flight, so no launch is spent on it.
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

// The same products with the input quad already unpacked to F32 (an input
// reused across rows is then unpacked once, not once per row).
__device__ __forceinline__ void quad_acc_f(Quad& a, const float (&xl)[4], const float (&xh)[4],
                                           const u32x4& w) {
  a.lo[0] += xl[0] * lo2f(w.x); a.hi[0] += xh[0] * hi2f(w.x);
  a.lo[1] += xl[1] * lo2f(w.y); a.hi[1] += xh[1] * hi2f(w.y);
  a.lo[2] += xl[2] * lo2f(w.z); a.hi[2] += xh[2] * hi2f(w.z);
  a.lo[3] += xl[3] * lo2f(w.w); a.hi[3] += xh[3] * hi2f(w.w);
}

__device__ __forceinline__ void quad_unpack(const u32x4& x, float (&xl)[4], float (&xh)[4]) {
  xl[0] = lo2f(x.x); xh[0] = hi2f(x.x);
  xl[1] = lo2f(x.y); xh[1] = hi2f(x.y);
  xl[2] = lo2f(x.z); xh[2] = hi2f(x.z);
  xl[3] = lo2f(x.w); xh[3] = hi2f(x.w);
}

// Value of lane i + S as seen from lane i, for the lanes a tree level uses:
// S <= 8 within a 16-lane row (DPP row shift; lanes past the row end read
// +0 and are never used), S = 16 for rows 0 and 2 (permlane16 swap), S = 32
// for lanes 0-31 (permlane32 swap). No LDS traffic, unlike a bpermute.
template <int S>
__device__ __forceinline__ float lane_down(float v) {
  const int b = __builtin_bit_cast(int, v);
  if constexpr (S == 32) {
    return __builtin_bit_cast(float, (int)__builtin_amdgcn_permlane32_swap(b, b, false, false)[1]);
  } else if constexpr (S == 16) {
    return __builtin_bit_cast(float, (int)__builtin_amdgcn_permlane16_swap(b, b, false, false)[1]);
  } else {
    static_assert(S == 1 || S == 2 || S == 4 || S == 8, "DPP row shift");
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x100 + S, 0xf, 0xf, true));
  }
}

// Halving tree over 64 reference lanes held one per physical lane
// (strides 32 ... 1); result in lane 0.
__device__ __forceinline__ float tree64_lanes(float v) {
  v += lane_down<32>(v);
  v += lane_down<16>(v);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  v += lane_down<1>(v);
  return v;
}
// Halving tree over 32 reference lanes per half wave (strides 16 ... 1);
// results in lanes 0 and 32.
__device__ __forceinline__ float tree32_lanes(float v) {
  v += lane_down<16>(v);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  v += lane_down<1>(v);
  return v;
}

// Two such trees at once: a's total in lane 0 of each half wave, b's in
// lane 16. At stride 16 one permlane16 swap of a with b leaves a's two rows
// side by side in rows 0 and 2 (the first result holds a's even rows, the
// second a's odd rows there) and b's in rows 1 and 3, so one add gives a's
// stride-16 sums in lanes 0-15 of a half and b's in lanes 16-31; strides
// 8 ... 1 then run inside each 16-lane row. Every sum has the operands it
// has in tree32_lanes (a sum's operands commute), so both totals are its
// bits.
__device__ __forceinline__ float tree32_pair(float a, float b) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, a), __builtin_bit_cast(int, b), false,
                                                  false);
  float v = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  v += lane_down<1>(v);
  return v;
}

// Halving tree of width W = 4*LPR over the reference lanes held by the LPR
// physical lanes of a row group (reference stride 4s = physical stride s,
// then strides 2 and 1 inside the lane). Must be reached by every lane of
// the wave. The result is valid in the group's first lane.
template <int LPR, int S = LPR / 2>
__device__ __forceinline__ void tree_levels(float& v0, float& v1, float& v2, float& v3) {
  if constexpr (S >= 1) {
    v0 += lane_down<S>(v0);
    v1 += lane_down<S>(v1);
    v2 += lane_down<S>(v2);
    v3 += lane_down<S>(v3);
    tree_levels<LPR, S / 2>(v0, v1, v2, v3);
  }
}

template <int LPR>
__device__ __forceinline__ float quad_tree(const Quad& a) {
  float v0 = a.lo[0] + a.hi[0];
  float v1 = a.lo[1] + a.hi[1];
  float v2 = a.lo[2] + a.hi[2];
  float v3 = a.lo[3] + a.hi[3];
  tree_levels<LPR>(v0, v1, v2, v3);
  v0 += v2;
  v1 += v3;
  return v0 + v1;
}

// Two quad_tree<64> totals at once: a's in lane 31, b's in lane 63. The
// first level (physical stride 32) is one permlane32 swap per value: the
// lower half receives a's upper values, the upper half b's lower ones, so
// lanes 0-31 continue a's tree and lanes 32-63 b's. At stride 16, v0 and v1
// (and v2 and v3) share one permlane16 swap: rows 0 and 2 go on with v0's
// (v2's) tree, rows 1 and 3 with v1's (v3's), no copies needed. Strides
// 8 ... 1 then add lane i - s into lane i (the sum of reference lanes j and
// j + s lands in the later one, with the same two operands), so each row's
// total ends in its last lane: v0 + v2 in lanes 15 and 47, v1 + v3 in lanes
// 31 and 63, and a row-15 broadcast adds them. Every sum has quad_tree<64>'s
// operands (the two operands of a sum commute): the same bits in far fewer
// instructions.
// The same tree over four values per lane held directly (the B256 order's
// per-lane sums): a's total in lane 31, b's in lane 63.
__device__ __forceinline__ float tree64_pair4_end(const float (&a)[4], const float (&b)[4]) {
  float v[4];
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(int, a[p]), __builtin_bit_cast(int, b[p]), false,
                                                    false);
    v[p] = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
  float w[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(int, v[2 * q]),
                                                    __builtin_bit_cast(int, v[2 * q + 1]), false, false);
    w[q] = __builtin_bit_cast(float, (int)r[0]) + __builtin_bit_cast(float, (int)r[1]);
  }
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    int b = __builtin_bit_cast(int, w[q]);
    w[q] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x118, 0xf, 0xf, true));  // row_shr:8
    b = __builtin_bit_cast(int, w[q]);
    w[q] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x114, 0xf, 0xf, true));  // row_shr:4
    b = __builtin_bit_cast(int, w[q]);
    w[q] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x112, 0xf, 0xf, true));  // row_shr:2
    b = __builtin_bit_cast(int, w[q]);
    w[q] += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, b, 0x111, 0xf, 0xf, true));  // row_shr:1
  }
  const float s = w[0] + w[1];
  // row_bcast:15 (lane 15 of each row to the next row; rows 1 and 3 are the
  // ones read)
  return s + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x142, 0xf, 0xf, true));
}
__device__ __forceinline__ float quad_tree64_pair_end(const Quad& a, const Quad& b) {
  const float av[4] = {a.lo[0] + a.hi[0], a.lo[1] + a.hi[1], a.lo[2] + a.hi[2], a.lo[3] + a.hi[3]};
  const float bv[4] = {b.lo[0] + b.hi[0], b.lo[1] + b.hi[1], b.lo[2] + b.hi[2], b.lo[3] + b.hi[3]};
  return tree64_pair4_end(av, bv);
}

// The value lane `lane` holds, in every lane (a scalar read).
__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

__device__ __forceinline__ u32x4 ldq(const void* base, int64_t quad) {
  return reinterpret_cast<const u32x4*>(base)[quad];
}

__device__ __forceinline__ uint32_t pack_bf(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// ------------------------------------------------------------ input staging

// qwen35.normalize (qwen35.hex:912-977) of one row of `cols` BF16 values into
// LDS as packed BF16 quads: y_i = bf16(bf16(x_i * inv) * bf16(w_i)),
// inv = 1 / sqrt(S / cols + eps), S the adjacent-pair tree sum of the squares
// over the next power of two `pad` >= cols (zero padded).
//
// cols <= 2048 (every preset): thread t owns octet t (8 values), loaded by
// norm_prefetch before the caller's weight loads. An in-register tree over
// the octet, a shuffle tree over the 64 lanes of a wave and
// ((w0 + w1) + (w2 + w3)) over the waves; threads past pad/8 hold +0, and
// joining a subtotal with a zero subtree is exact, so the result equals the
// tree over pad. Wider rows (up to 16384) take a generic path in which thread
// t owns pad/2048 consecutive octets. Requires blockDim.x == 256.
struct NormIn {
  u32x4 x;
  f32x4 w0, w1;
};

__device__ __forceinline__ void norm_prefetch(NormIn& in, const uint16_t* __restrict__ x,
                                              const float* __restrict__ w, int cols) {
  const int o = min((int)threadIdx.x, (cols >> 3) - 1);
  in.x = ldq(x, o);
  in.w0 = reinterpret_cast<const f32x4*>(w)[2 * o];
  in.w1 = reinterpret_cast<const f32x4*>(w)[2 * o + 1];
}

__device__ __forceinline__ float octet_squares(const u32x4& v) {
  const float s0 = lo2f(v.x) * lo2f(v.x), s1 = hi2f(v.x) * hi2f(v.x);
  const float s2 = lo2f(v.y) * lo2f(v.y), s3 = hi2f(v.y) * hi2f(v.y);
  const float s4 = lo2f(v.z) * lo2f(v.z), s5 = hi2f(v.z) * hi2f(v.z);
  const float s6 = lo2f(v.w) * lo2f(v.w), s7 = hi2f(v.w) * hi2f(v.w);
  return ((s0 + s1) + (s2 + s3)) + ((s4 + s5) + (s6 + s7));
}

__device__ __forceinline__ u32x4 octet_scale(const u32x4& v, float inverse, const f32x4& w0,
                                             const f32x4& w1) {
  u32x4 y;
  y.x = pack_bf(bf_mul(f2bf(lo2f(v.x) * inverse), f2bf(w0.x)),
                bf_mul(f2bf(hi2f(v.x) * inverse), f2bf(w0.y)));
  y.y = pack_bf(bf_mul(f2bf(lo2f(v.y) * inverse), f2bf(w0.z)),
                bf_mul(f2bf(hi2f(v.y) * inverse), f2bf(w0.w)));
  y.z = pack_bf(bf_mul(f2bf(lo2f(v.z) * inverse), f2bf(w1.x)),
                bf_mul(f2bf(hi2f(v.z) * inverse), f2bf(w1.y)));
  y.w = pack_bf(bf_mul(f2bf(lo2f(v.w) * inverse), f2bf(w1.z)),
                bf_mul(f2bf(hi2f(v.w) * inverse), f2bf(w1.w)));
  return y;
}

// Thread-total -> block-total: shuffle tree over the wave, then the waves.
__device__ __forceinline__ float block_ap_sum(float t, float* red) {
  t = t + lane_down<1>(t);
  t = t + lane_down<2>(t);
  t = t + lane_down<4>(t);
  t = t + lane_down<8>(t);
  t = t + lane_down<16>(t);
  t = t + lane_down<32>(t);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = t;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

__device__ __noinline__ void norm_wide(u32x4* xs, const uint16_t* __restrict__ x,
                                       const float* __restrict__ w, int cols, float eps,
                                       float* red) {
  const int tid = threadIdx.x, octs = cols >> 3;
  int pad = 8;
  while (pad < cols) pad <<= 1;
  const int m = pad >> 11;  // 2..8 octets per thread
  float part[8];
  for (int j = 0; j < 8; ++j) {
    const int o = tid * m + j;
    part[j] = (j < m && o < octs) ? octet_squares(ldq(x, o)) : 0.0f;
  }
  for (int d = 1; d < m; d <<= 1)
    for (int j = 0; j + d < m; j += 2 * d) part[j] = part[j] + part[j + d];
  const float sum = block_ap_sum(part[0], red);
  const float inverse = 1.0f / nsqrt(sum / (float)cols + eps);
  for (int j = 0; j < m; ++j) {
    const int o = tid * m + j;
    if (o < octs)
      xs[o] = octet_scale(ldq(x, o), inverse, reinterpret_cast<const f32x4*>(w)[2 * o],
                          reinterpret_cast<const f32x4*>(w)[2 * o + 1]);
  }
  __syncthreads();
}

__device__ __forceinline__ void norm_finish(const NormIn& in, u32x4* xs,
                                            const uint16_t* __restrict__ x,
                                            const float* __restrict__ w, int cols, float eps,
                                            float* red) {
  if (cols > 2048) {
    norm_wide(xs, x, w, cols, eps, red);
    return;
  }
  const bool own = (int)threadIdx.x < (cols >> 3);
  const float sum = block_ap_sum(own ? octet_squares(in.x) : 0.0f, red);
  const float inverse = 1.0f / nsqrt(sum / (float)cols + eps);
  if (own) xs[threadIdx.x] = octet_scale(in.x, inverse, in.w0, in.w1);
  __syncthreads();
}

// Plain copy of a BF16 row (already in its final form) into LDS: kXQ quads
// per thread prefetched into registers, any remainder copied afterwards.
template <int kXQ>
struct CopyIn {
  u32x4 v[kXQ];
};

template <int kXQ>
__device__ __forceinline__ void copy_prefetch(CopyIn<kXQ>& in, const uint16_t* __restrict__ x,
                                              int cols) {
  const int quads = cols >> 3;
#pragma unroll
  for (int j = 0; j < kXQ; ++j) in.v[j] = ldq(x, min((int)(threadIdx.x + blockDim.x * j), quads - 1));
}

template <int kXQ>
__device__ __forceinline__ void copy_finish(const CopyIn<kXQ>& in, u32x4* xs,
                                            const uint16_t* __restrict__ x, int cols) {
  const int quads = cols >> 3;
#pragma unroll
  for (int j = 0; j < kXQ; ++j) {
    const int i = threadIdx.x + blockDim.x * j;
    if (i < quads) xs[i] = in.v[j];
  }
  for (int i = threadIdx.x + blockDim.x * kXQ; i < quads; i += blockDim.x) xs[i] = ldq(x, i);
  __syncthreads();
}

// ---------------------------------------------------------- S256 projection

// Up to four row-major matrices sharing one input (group-project,
// group_projection.hex:3-97). Rows are numbered across segments.
struct Segments {
  const uint16_t* w[4];
  uint16_t* out[4];
  int rows[4];
  int count;
};

// Segment of a row and its row within the segment; selects rather than an
// indexed kernel-argument load, so the weight address is ready at once.
__device__ __forceinline__ int segment_of(const Segments& seg, int row, int* local) {
  const int e0 = seg.rows[0], e1 = e0 + seg.rows[1], e2 = e1 + seg.rows[2];
  const int s = row < e0 ? 0 : row < e1 ? 1 : row < e2 ? 2 : 3;
  *local = row - (s == 0 ? 0 : s == 1 ? e0 : s == 2 ? e1 : e2);
  return s;
}
__device__ __forceinline__ const uint16_t* segment_w(const Segments& seg, int s) {
  return s == 0 ? seg.w[0] : s == 1 ? seg.w[1] : s == 2 ? seg.w[2] : seg.w[3];
}
__device__ __forceinline__ uint16_t* segment_out(const Segments& seg, int s) {
  return s == 0 ? seg.out[0] : s == 1 ? seg.out[1] : s == 2 ? seg.out[2] : seg.out[3];
}

// S256 (64 lanes per row): each wave streams kRows256 rows, each lane four
// quads of each per batch (cols <= 2048 is one batch). Output bf16 of the
// tree (simt.hex:400-410). kNorm: the input is the hidden row normalised in
// the prologue; otherwise it is used as given. Held to 128 VGPRs so four
// blocks fit per CU and a 12352-row DeltaNet projection runs in one round.
constexpr int kRows256 = 4;

template <bool kNorm>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(4))) void k_project256(const uint16_t* __restrict__ x,
                                                        const float* __restrict__ norm_w, float eps,
                                                        Segments seg, int cols) {
  constexpr int RW = kRows256, NQ = 4;
  extern __shared__ __align__(16) u32x4 xs[];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quads = cols >> 3;
  const int total = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int row0 = (blockIdx.x * 4 + wave) * RW;
  NormIn nin;
  CopyIn<1> cin;
  if (kNorm) norm_prefetch(nin, x, norm_w, cols);
  else copy_prefetch(cin, x, cols);
  // Row r's weights; recomputed for later batches so no pointer stays live.
  auto row_w = [&](int r) {
    int local;
    const int s = segment_of(seg, min(row0 + r, total - 1), &local);
    return segment_w(seg, s) + (size_t)local * cols;
  };
  u32x4 wv[RW][NQ];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const uint16_t* wr = row_w(r);
#pragma unroll
    for (int j = 0; j < NQ; ++j) wv[r][j] = ldq(wr, min(lane + 64 * j, quads - 1));
  }
  if (kNorm) norm_finish(nin, xs, x, norm_w, cols, eps, red);
  else copy_finish(cin, xs, x, cols);
  u32x4 xq[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) xq[j] = xs[min(lane + 64 * j, quads - 1)];
  // One row at a time: row r's tree overlaps the arrival of row r+1.
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    Quad acc;
    quad_zero(acc);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (lane + 64 * j < quads) quad_acc(acc, xq[j], wv[r][j]);
    // Rows wider than 64 * NQ quads (hidden > 2048): remaining batches.
    for (int b = 1; b * 64 * NQ < quads; ++b) {
      const uint16_t* wr = row_w(r);
#pragma unroll
      for (int j = 0; j < NQ; ++j) wv[r][j] = ldq(wr, min(lane + 64 * (NQ * b + j), quads - 1));
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int qi = lane + 64 * (NQ * b + j);
        if (qi < quads) quad_acc(acc, xs[qi], wv[r][j]);
      }
    }
    const float v = quad_tree<64>(acc);
    if (lane == 0 && row0 + r < total) {
      int local;
      const int s = segment_of(seg, row0 + r, &local);
      segment_out(seg, s)[local] = f2bf(v);
    }
  }
}

// ------------------------------------------------------------ S32 projection

// S32 (8 lanes per row, 8 rows per wave, 32 per block): dense projections
// (simt.hex:400-410) and, with kArgmax, the vocabulary head fused with the
// greedy argmax (simt.hex:348-441 + fused_argmax.hex:1-104). kNQ quads per
// lane per batch; cols <= 64 * kNQ is one batch.

// Orderable key of a BF16 logit for a (value, first index) maximum: larger
// value wins, equal values prefer the lower index; -0 equals +0; NaN never
// wins. key 0 means "no candidate".
__device__ __forceinline__ unsigned long long logit_key(uint16_t b, uint32_t index) {
  float v = bf2f(b);
  if (v != v) return 0ull;
  uint32_t u = v == 0.0f ? 0u : fbits(v);
  uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return ((unsigned long long)ordered << 32) | (unsigned long long)(0xffffffffu - index);
}

template <bool kNorm, bool kArgmax, int kNQ>
__global__ __launch_bounds__(kBlock) void k_project32(const uint16_t* __restrict__ x,
                                                       const float* __restrict__ norm_w, float eps,
                                                       Segments seg, int cols,
                                                       unsigned long long* __restrict__ best) {
  constexpr int NQ = kNQ;
  extern __shared__ __align__(16) u32x4 xs[];
  __shared__ float red[4];
  __shared__ unsigned long long wave_best[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int q = lane & 7, g = lane >> 3;
  const int quads = cols >> 3;
  const int total = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int row = (blockIdx.x * 4 + wave) * 8 + g;
  NormIn nin;
  CopyIn<1> cin;
  if (kNorm) norm_prefetch(nin, x, norm_w, cols);
  else copy_prefetch(cin, x, cols);
  int local;
  const int s = segment_of(seg, min(row, total - 1), &local);
  const uint16_t* wr = segment_w(seg, s) + (size_t)local * cols;
  u32x4 wv[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, min(q + 8 * j, quads - 1));
  if (kNorm) norm_finish(nin, xs, x, norm_w, cols, eps, red);
  else copy_finish(cin, xs, x, cols);
  Quad acc;
  quad_zero(acc);
  for (int b = 0; b * 8 * NQ < quads; ++b) {
    if (b > 0) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, min(q + 8 * (NQ * b + j), quads - 1));
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int qi = q + 8 * (NQ * b + j);
      if (qi < quads) quad_acc(acc, xs[qi], wv[j]);
    }
  }
  const float v = quad_tree<8>(acc);
  unsigned long long mine = 0ull;
  if (q == 0 && row < total) {
    const uint16_t b = f2bf(v);
    segment_out(seg, s)[local] = b;
    if (kArgmax) mine = logit_key(b, (uint32_t)row);
  }
  if (kArgmax) {
#pragma unroll
    for (int d = 32; d >= 8; d >>= 1) {
      const unsigned long long o = __shfl_down(mine, d, 64);
      mine = o > mine ? o : mine;
    }
    if (lane == 0) wave_best[wave] = mine;
    __syncthreads();
    if (threadIdx.x == 0) {
      unsigned long long b = wave_best[0];
#pragma unroll
      for (int i = 1; i < 4; ++i) b = wave_best[i] > b ? wave_best[i] : b;
      if (b) atomicMax(best, b);
    }
  }
}

// ------------------------------------------------------- S64 residual output

// bf16(bf16(tree64(x . w_r)) (+) res_r) (qwen3.fused.residual,
// simt.hex:442-538), or bf16(tree64) when res is null. One wave per block,
// four rows per wave (16 lanes per row); kNQ quads per lane per batch
// (cols <= 128 * kNQ is one batch, and then the input fits the prefetch).
template <int kNQ>
__global__ __launch_bounds__(64) void k_residual(const uint16_t* __restrict__ x,
                                                  const uint16_t* __restrict__ w, int rows,
                                                  int cols, const uint16_t* __restrict__ res,
                                                  uint16_t* __restrict__ out) {
  constexpr int NQ = kNQ;
  extern __shared__ __align__(16) u32x4 xs[];
  const int lane = threadIdx.x, q = lane & 15, g = lane >> 4;
  const int quads = cols >> 3;
  const int row = blockIdx.x * 4 + g;
  CopyIn<NQ / 4> cin;
  copy_prefetch(cin, x, cols);
  const uint16_t* wr = w + (size_t)min(row, rows - 1) * cols;
  u32x4 wv[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, min(q + 16 * j, quads - 1));
  const uint16_t rv = (q == 0 && res) ? res[min(row, rows - 1)] : (uint16_t)0;
  copy_finish(cin, xs, x, cols);
  Quad acc;
  quad_zero(acc);
  for (int b = 0; b * 16 * NQ < quads; ++b) {
    if (b > 0) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) wv[j] = ldq(wr, min(q + 16 * (NQ * b + j), quads - 1));
    }
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const int qi = q + 16 * (NQ * b + j);
      if (qi < quads) quad_acc(acc, xs[qi], wv[j]);
    }
  }
  const float v = quad_tree<16>(acc);
  if (q == 0 && row < rows) out[row] = res ? bf_add(f2bf(v), rv) : f2bf(v);
}

// ------------------------------------------------------------- MoE router

// Router (moe.hex:4-84) over the normalised hidden row with F32 weights:
// rows [0, E) routed, row E the shared-expert gate; S32, F32 logits. One
// wave per row; physical lane l = 2r + h runs reference lane r's low (h = 0)
// or high (h = 1) accumulator over floats 64k + l, k = 0, 1, ... (64
// coalesced dwords per step), then lo + hi and the halving tree.
//
// The last block to finish (atomic ticket after a device-scope fence) ranks
// the routed logits, rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)},
// and writes the top-k ids in rank order with their softmax weights
// p_j = exp(l_j - l_0) / sum exp (moe.hex:86-252), then resets the ticket.
template <int kND>
__global__ __launch_bounds__(kBlock) void k_router_select(
    const uint16_t* __restrict__ x, const float* __restrict__ norm_w, float eps, int cols,
    const float* __restrict__ w, const float* __restrict__ shared_w, int experts, int top_k,
    float* __restrict__ logits, int* __restrict__ ids, float* __restrict__ probs,
    unsigned* __restrict__ ticket) {
  constexpr int ND = kND;
  extern __shared__ __align__(16) u32x4 xs[];
  __shared__ float red[4];
  __shared__ float chosen[64];
  __shared__ int last;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = experts + 1;
  const int row = blockIdx.x * 4 + wave;
  const int rc = min(row, rows - 1);
  NormIn nin;
  norm_prefetch(nin, x, norm_w, cols);
  const float* wr = rc < experts ? w + (size_t)rc * cols : shared_w;
  float wv[ND];
#pragma unroll
  for (int j = 0; j < ND; ++j) wv[j] = wr[min(64 * j + lane, cols - 1)];
  norm_finish(nin, xs, x, norm_w, cols, eps, red);
  const uint16_t* xe = reinterpret_cast<const uint16_t*>(xs);
  float acc = 0.0f;
  for (int b = 0; b * 64 * ND < cols; ++b) {
    if (b > 0) {
#pragma unroll
      for (int j = 0; j < ND; ++j) wv[j] = wr[min(64 * (ND * b + j) + lane, cols - 1)];
    }
#pragma unroll
    for (int j = 0; j < ND; ++j) {
      const int i = 64 * (ND * b + j) + lane;
      if (i < cols) acc += bf2f(xe[i]) * wv[j];
    }
  }
  // lane 2r: lo_r + hi_r, then reference strides 16..1 = physical 32..2
  float v = acc + lane_down<1>(acc);
  v += lane_down<32>(v);
  v += lane_down<16>(v);
  v += lane_down<8>(v);
  v += lane_down<4>(v);
  v += lane_down<2>(v);
  if (lane == 0 && row < rows)
    __hip_atomic_store(logits + row, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);

  // The logits went out as device-coherent stores. Every wave releases its
  // own stores at device scope (waits until they have completed), then one
  // ticket per block tells the last block it may read them all; that block
  // acquires at device scope before its reads.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  __syncthreads();
  if (threadIdx.x == 0)
    last = __hip_atomic_fetch_add(ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) ==
           gridDim.x - 1;
  __syncthreads();
  if (!last) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  float* lg = reinterpret_cast<float*>(xs);  // the staged row is no longer needed
  __shared__ int any_nan;
  if (threadIdx.x == 0) any_nan = 0;
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += blockDim.x) {
    const float le = __hip_atomic_load(logits + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    lg[e] = le;
    if (le != le) any_nan = 1;
  }
  __syncthreads();
  if (!any_nan) {
    // Without NaNs the rank order is the stable descending order: top_k
    // rounds of a wave-wide maximum of (value, lowest index) keys.
    if (wave == 0) {
      unsigned long long taken = 0;  // bit j: lane's j-th candidate chosen (experts <= 4096)
      for (int k = 0; k < top_k; ++k) {
        unsigned long long mine = 0ull;
        for (int j = 0, e = lane; e < experts; ++j, e += 64) {
          if ((taken >> j) & 1ull) continue;
          const float le = lg[e];
          const uint32_t u = le == 0.0f ? 0u : fbits(le);
          const uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
          const unsigned long long key =
              ((unsigned long long)ordered << 32) | (0xffffffffu - (uint32_t)e);
          mine = key > mine ? key : mine;
        }
        unsigned long long best = mine;
#pragma unroll
        for (int s = 32; s >= 1; s >>= 1) {
          const unsigned long long o = __shfl_xor(best, s, 64);
          best = o > best ? o : best;
        }
        const int e = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
        if ((e & 63) == lane) taken |= 1ull << (e >> 6);
        if (lane == 0) {
          ids[k] = e;
          chosen[k] = lg[e];
        }
      }
    }
  } else {
    // rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)}. With NaNs two
    // experts can share a rank and leave another unassigned: the largest
    // expert index of a shared rank takes it (the restatement's ascending
    // scatter; an LDS maximum), an unassigned rank k keeps expert k.
    __shared__ int won[64];
    if (threadIdx.x < top_k) won[threadIdx.x] = -1;
    __syncthreads();
    for (int e = threadIdx.x; e < experts; e += blockDim.x) {
      const float le = lg[e];
      int rank = 0;
      for (int i = 0; i < experts; ++i) {
        const float o = lg[i];
        rank += (o > le) ? 1 : ((i < e && !(le > o)) ? 1 : 0);
      }
      if (rank < top_k) atomicMax(&won[rank], e);
    }
    __syncthreads();
    if (threadIdx.x < top_k) {
      const int e = won[threadIdx.x] >= 0 ? won[threadIdx.x] : threadIdx.x;
      ids[threadIdx.x] = e;
      chosen[threadIdx.x] = lg[e];
    }
  }
  __syncthreads();
  if (wave == 0) {
    // p_j = exp(l_j - l_0) / den, den summed left to right from 0.
    const float ex = lane < top_k ? hexp(chosen[lane] - chosen[0]) : 0.0f;
    float den = 0.0f;
    for (int j = 0; j < top_k; ++j) den = den + __shfl(ex, j, 64);
    if (lane < top_k) probs[lane] = ex / den;
    if (lane == 0) __hip_atomic_store(ticket, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

inline size_t router_lds_bytes(int cols, int experts) {
  return (size_t)(cols * 2 > experts * 4 ? cols * 2 : experts * 4);
}

// ------------------------------------------------------ dual S256 (SwiGLU)

// Routed + shared expert gate/up (moe.hex:254-333) or the dense SwiGLU
// (qwen3.fused.gate, simt.hex:539-646) over the normalised hidden row.
// MoE rows [0, K*I) belong to the selected experts in rank order, rows
// [K*I, K*I+SI) to the shared expert. Routed: bf16(silu(g) * u * p_slot);
// shared: bf16(bf16(bf16(silu(g)) * u) * sigmoid(shared logit)); dense:
// bf16(bf16(silu(bf16 g)) * bf16(u)). kRowsGate rows per wave (at the
// 35B-A3B shape 9216 rows = 768 blocks, one per resident slot).
constexpr int kRowsGate = 3;

template <bool kMoE>
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(3))) void k_gate_up(
    const uint16_t* __restrict__ x, const float* __restrict__ norm_w, float eps, int cols,
    const uint16_t* __restrict__ gate, const uint16_t* __restrict__ up,
    const uint16_t* __restrict__ sgate, const uint16_t* __restrict__ sup,
    const int* __restrict__ ids, const float* __restrict__ probs,
    const float* __restrict__ router, int experts, int top_k, int inter, int shared_inter,
    uint16_t* __restrict__ active) {
  constexpr int RW = kRowsGate, NQ = 4;
  extern __shared__ __align__(16) u32x4 xs[];
  __shared__ float red[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quads = cols >> 3;
  const int routed_rows = kMoE ? top_k * inter : inter;
  const int rows = kMoE ? routed_rows + shared_inter : inter;
  const int row0 = (blockIdx.x * 4 + wave) * RW;
  NormIn nin;
  norm_prefetch(nin, x, norm_w, cols);
  // Gate and up rows of row r (recomputed for later batches so no pointer
  // stays live).
  auto row_ptrs = [&](int r, const uint16_t*& g, const uint16_t*& u) {
    const int row = min(row0 + r, rows - 1);
    if (!kMoE) {
      g = gate + (size_t)row * cols;
      u = up + (size_t)row * cols;
    } else if (row < routed_rows) {
      const int slot = row / inter;
      const size_t e = (size_t)ids[slot] * inter + (row - slot * inter);
      g = gate + e * cols;
      u = up + e * cols;
    } else {
      g = sgate + (size_t)(row - routed_rows) * cols;
      u = sup + (size_t)(row - routed_rows) * cols;
    }
  };
  u32x4 gv[RW][NQ], uv[RW][NQ];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    const uint16_t *wg, *wu;
    row_ptrs(r, wg, wu);
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      gv[r][j] = ldq(wg, min(lane + 64 * j, quads - 1));
      uv[r][j] = ldq(wu, min(lane + 64 * j, quads - 1));
    }
  }
  norm_finish(nin, xs, x, norm_w, cols, eps, red);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    Quad ga, ua;
    quad_zero(ga);
    quad_zero(ua);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (lane + 64 * j < quads) {
        const u32x4 xq = xs[lane + 64 * j];
        quad_acc(ga, xq, gv[r][j]);
        quad_acc(ua, xq, uv[r][j]);
      }
    for (int b = 1; b * 64 * NQ < quads; ++b) {  // hidden > 2048
      const uint16_t *wg, *wu;
      row_ptrs(r, wg, wu);
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        gv[r][j] = ldq(wg, min(lane + 64 * (NQ * b + j), quads - 1));
        uv[r][j] = ldq(wu, min(lane + 64 * (NQ * b + j), quads - 1));
      }
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const int qi = lane + 64 * (NQ * b + j);
        if (qi < quads) {
          quad_acc(ga, xs[qi], gv[r][j]);
          quad_acc(ua, xs[qi], uv[r][j]);
        }
      }
    }
    const float gsum = quad_tree<64>(ga);
    const float usum = quad_tree<64>(ua);
    const int row = row0 + r;
    if (lane == 0 && row < rows) {
      if (!kMoE) {
        active[row] = bf_mul(f2bf(silu(rbf(gsum))), f2bf(usum));
      } else {
        const float gb = rbf(gsum), ub = rbf(usum);
        const float activated = silu(gb);
        float y;
        if (row < routed_rows) y = (activated * ub) * probs[row / inter];
        else y = rbf(rbf(activated) * ub) * sigmoid(router[experts]);
        active[row] = f2bf(y);
      }
    }
  }
}

// ----------------------------------------------------- MoE down projection

// Expert down projection (moe.hex:371-434, simt_moe.hex:36-287): per hidden
// row, S32 over the concatenated routed activations (pair p reads expert
// ids[p / (I/2)]) and a separate S32 over the shared activations;
// out = bf16(bf16(routed + residual) (+) bf16(shared)).
//
// A row's chains (72 quads per reference-lane group at the 35B shape) are
// too long to stream from registers, so the block stages kDownRows rows in
// LDS: wave w loads row row0 + w with all 64 lanes (kNQ quads each, all in
// flight; a row is at most 64 * kNQ quads), then wave 0 reduces the rows from
// LDS in the reference order (8 lanes per row).
constexpr int kDownRows = 4;

template <int kNQ>
__global__ __launch_bounds__(kBlock) void k_moe_down(
    const uint16_t* __restrict__ active, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ sdown, const int* __restrict__ ids,
    const uint16_t* __restrict__ residual, int hidden, int top_k, int inter, int shared_inter,
    uint16_t* __restrict__ out) {
  constexpr int NQ = kNQ;
  extern __shared__ __align__(16) u32x4 sm[];
  const int rq = top_k * inter / 8, sq = shared_inter / 8, per_row = rq + sq;
  const int iq = inter / 8;
  const int per_row_cols = per_row * 8;
  u32x4* xs = sm;
  u32x4* ws = sm + per_row;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int row0 = blockIdx.x * kDownRows;
  const int row = min(row0 + wave, hidden - 1);
  CopyIn<NQ / 4> cin;
  copy_prefetch(cin, active, per_row_cols);
  int slot_id[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int k = min(lane + 64 * j, rq - 1);
    slot_id[j] = ids[k / iq];
  }
  u32x4 wv[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int k = min(lane + 64 * j, per_row - 1);
    const int slot = min(k, rq - 1) / iq;
    const u32x4* src =
        k < rq ? reinterpret_cast<const u32x4*>(down + ((size_t)slot_id[j] * hidden + row) * inter) +
                     (k - slot * iq)
               : reinterpret_cast<const u32x4*>(sdown + (size_t)row * shared_inter) + (k - rq);
    wv[j] = *src;
  }
  copy_finish(cin, xs, active, per_row_cols);
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int k = lane + 64 * j;
    if (k < per_row) ws[wave * per_row + k] = wv[j];
  }
  __syncthreads();
  if (wave == 0) {
    const int g = lane >> 3, q = lane & 7;
    const int nrows = min(kDownRows, hidden - row0);
    Quad r, s;
    quad_zero(r);
    quad_zero(s);
    if (g < nrows) {
      const u32x4* wr = ws + g * per_row;
      for (int i = q; i < rq; i += 8) quad_acc(r, xs[i], wr[i]);
      for (int i = q; i < sq; i += 8) quad_acc(s, xs[rq + i], wr[rq + i]);
    }
    const float rv = quad_tree<8>(r);
    const float sv = quad_tree<8>(s);
    if (q == 0 && g < nrows) {
      const int o = row0 + g;
      out[o] = bf_add(f2bf(rv + bf2f(residual[o])), f2bf(sv));
    }
  }
}

inline size_t moe_down_lds_bytes(int per_row_quads) {
  return (size_t)(1 + kDownRows) * per_row_quads * 16;
}

}  // namespace cq35
