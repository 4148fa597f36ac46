// Matrix-core prefill: the reference's matrix-core prompt path (wmma_prefill,
// qwen35.rs:467-541 with the grouped-expert and projection stages of
// qwen35_wmma_moe.hex) on CDNA4 MFMA. The products are the same as the
// batched SIMT projections (prefill.h) but the F32 accumulation runs inside
// v_mfma_f32_32x32x16_bf16, whose summation order is the hardware's: results
// agree with the exact path to accumulation rounding, not bit for bit, as
// the reference's own matrix-core path does (README.md:59-60). The exact
// SIMT path stays the default; a session selects this one per component.
//
// Operand layouts of v_mfma_f32_32x32x16_bf16 (checked on the device): lane
// l supplies A[l % 32][8 (l / 32) + i] and B[8 (l / 32) + i][l % 32] for
// i < 8, and receives D[8 (r / 4) + 4 (l / 32) + r % 4][l % 32] in
// accumulator register r < 16. Both prefill operands are K-contiguous
// (activations [token][k], weights [row][k]), so every fragment is one
// 16-byte load.
#pragma once

#include "prefill.h"

namespace cq35 {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ f32x16_t mfma32(const u32x4& a, const u32x4& b, const f32x16_t& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

constexpr int kMTokens = 32;             // tokens per wave tile
constexpr int kMRows = 64;               // weight rows per block tile (two 32-row MFMA tiles)
constexpr int kMWaves = 4;               // waves per block, along tokens
constexpr int kMBlockTokens = kMTokens * kMWaves;

// out[t][row] = epilogue(sum_k x[t][k] w[row][k]) for t < n, row < rows;
// cols % 16 == 0. Block (row tile bx, token tile by); wave w takes tokens
// [128 by + 32 w, +32). k steps of 16 rotate over kParts independent partial
// sums, added as a tree at the end: shorter F32 chains than one running
// accumulator (closer to the reference's lane-partials-then-tree orders) and
// independent MFMA dependency chains. The epilogues are those of k_bproject:
// bf16(total); bf16(total) (+) res; bf16(silu(bf16 g)) (x) bf16(u) with u
// from w2.
template <int kMode>
__global__ __launch_bounds__(64 * kMWaves) void k_mproject(const uint16_t* __restrict__ x, int n, int cols,
                                                           const uint16_t* __restrict__ w,
                                                           const uint16_t* __restrict__ w2, int rows,
                                                           const uint16_t* __restrict__ res,
                                                           uint16_t* __restrict__ out) {
  constexpr int kParts = kMode == kBGate ? 2 : 4;
  constexpr int kMats = kMode == kBGate ? 2 : 1;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t0 = blockIdx.y * kMBlockTokens + wave * kMTokens;
  if (t0 >= n) return;  // uniform per wave; no barriers below
  const int r0 = blockIdx.x * kMRows;
  const int kq = 8 * (lane >> 5);  // this lane's k offset inside a 16-wide step
  const int tr = min(t0 + (lane & 31), n - 1);
  const uint16_t* xa = x + (size_t)tr * cols + kq;
  const uint16_t* wp[kMats][2];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int wr = min(r0 + 32 * h + (lane & 31), rows - 1);
    wp[0][h] = w + (size_t)wr * cols + kq;
    if (kMode == kBGate) wp[kMats - 1][h] = w2 + (size_t)wr * cols + kq;
  }
  f32x16_t acc[kParts][kMats][2];
#pragma unroll
  for (int p = 0; p < kParts; ++p)
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi) acc[p][mi][0] = acc[p][mi][1] = f32x16_t{};
  const int steps = cols / 16;
  int st = 0;
  for (; st + kParts <= steps; st += kParts) {
    u32x4 a[kParts], b[kParts][kMats][2];
#pragma unroll
    for (int p = 0; p < kParts; ++p) {
      const int k = 16 * (st + p);
      a[p] = *reinterpret_cast<const u32x4*>(xa + k);
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) b[p][mi][h] = *reinterpret_cast<const u32x4*>(wp[mi][h] + k);
    }
#pragma unroll
    for (int p = 0; p < kParts; ++p)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[p][mi][h] = mfma32(a[p], b[p][mi][h], acc[p][mi][h]);
  }
  for (int p = 0; st < steps; ++st, ++p) {  // the last steps continue the rotation
    const int k = 16 * st;
    const u32x4 a = *reinterpret_cast<const u32x4*>(xa + k);
#pragma unroll
    for (int q = 0; q < kParts; ++q) {
      if (q != p) continue;
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h)
          acc[q][mi][h] = mfma32(a, *reinterpret_cast<const u32x4*>(wp[mi][h] + k), acc[q][mi][h]);
    }
  }
  // tree over the partial sums
#pragma unroll
  for (int span = 1; span < kParts; span *= 2)
#pragma unroll
    for (int p = 0; p + span < kParts; p += 2 * span)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[p][mi][h] += acc[p + span][mi][h];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = r0 + 32 * h + (lane & 31);
    if (row >= rows) continue;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = t0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (t >= n) continue;
      const size_t o = (size_t)t * rows + row;
      const float v = acc[0][0][h][r];
      uint16_t y;
      if (kMode == kBPlain) y = f2bf(v);
      else if (kMode == kBResidual) y = bf_add(f2bf(v), res[o]);
      else y = bf_mul(f2bf(silu(rbf(v))), f2bf(acc[0][kMats - 1][h][r]));
      out[o] = y;
    }
  }
}

// k_mproject's products with both operands staged through LDS, for cols a
// multiple of 128 (an even number of 64-column steps; other widths run
// k_mproject): block tile 128 tokens x 64 weight rows (wave w: tokens
// [32 w, +32) x the 64 rows, as k_mproject), K staged 64 columns per step,
// so a weight fragment is fetched
// once per block instead of once per wave. Global loads run two steps ahead
// of the multiplies (two register sets, three LDS buffers, one barrier per
// step): a step's loads have two steps' MFMA work to arrive in.
// The k steps of 16 go to the same rotating partial sums in the same order
// (step st of the row into part st % kParts, then the same tree), so every
// output is bit-identical to k_mproject's. LDS rows are 8 pieces of 16 bytes
// with piece p of row r stored in slot p ^ (r & 7): the 32 rows a fragment
// read touches spread over all banks. Blocks sharing a weight tile (all
// token tiles of one row tile) are placed on one XCD (block b runs on XCD
// b mod 8), so the tile is read from HBM once and from that XCD's L2 after.
constexpr int kGBK = 64;                // columns per LDS step
constexpr int kGPieces = kGBK / 8;      // 16-byte pieces per staged row
constexpr int kGTokens = kMBlockTokens;  // tokens per block tile
constexpr int kGBufs = 3;               // LDS buffers

__device__ __forceinline__ int gemm_slot(int row, int piece) { return row * kGPieces + (piece ^ (row & 7)); }

inline int gemm_grid(int rows, int n) {
  const int rt = (rows + kMRows - 1) / kMRows, tt = (n + kGTokens - 1) / kGTokens;
  return ((rt + 7) / 8) * 8 * tt;
}

template <int kMode>
struct GemmStage {
  static constexpr int kMats = kMode == kBGate ? 2 : 1;
  static constexpr int AP = kGTokens * kGPieces, BP = kMRows * kGPieces;  // pieces per stage
  static constexpr int kThreads = 64 * kMWaves;
  static constexpr int AL = AP / kThreads, BL = BP / kThreads;  // loads per thread per stage
  static_assert(AP % kThreads == 0 && BP % kThreads == 0, "stage loads");
  u32x4 a[AL], b[kMats][BL];
};

// The weight rows are the concatenation of up to four segments (matrix and
// output buffer each; row r of segment s goes to out_s[t][r]), so the
// projections of one input run as one launch; w2 (gate) and res (residual)
// go with a single segment.
template <int kMode>
__global__ __launch_bounds__(64 * kMWaves) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_mgemm(
    const uint16_t* __restrict__ x, int n, int cols, Segments seg, const uint16_t* __restrict__ w2,
    const uint16_t* __restrict__ res) {
  const int rows = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  using St = GemmStage<kMode>;
  constexpr int kParts = kMode == kBGate ? 2 : 4;
  constexpr int kMats = St::kMats, AP = St::AP, BP = St::BP, AL = St::AL, BL = St::BL;
  constexpr int kThreads = St::kThreads;
  __shared__ u32x4 sa[kGBufs][AP];
  __shared__ u32x4 sb[kGBufs][kMats][BP];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int tt = (n + kGTokens - 1) / kGTokens;
  const int b = blockIdx.x, xcd = b & 7, r = b >> 3;
  const int tile_t = r % tt, tile_r = (r / tt) * 8 + xcd;
  const int r0 = tile_r * kMRows;
  if (r0 >= rows) return;  // uniform per block
  const int tb = tile_t * kGTokens;
  // this thread's pieces of a stage: piece p = tid % 8 of rows tid / 8 +
  // 32 i (clamped rows); their LDS slots are slot0 + 256 i
  static_assert(kThreads % (8 * kGPieces) == 0, "one swizzle per thread");
  const int p8 = threadIdx.x % kGPieces, row8 = threadIdx.x / kGPieces;
  const int slot0 = gemm_slot(row8, p8);
  constexpr int kRowStep = kThreads / kGPieces;
  const uint16_t* ga[AL];
  const uint16_t* gb[kMats][BL];
#pragma unroll
  for (int i = 0; i < AL; ++i) ga[i] = x + (size_t)min(tb + row8 + kRowStep * i, n - 1) * cols + 8 * p8;
#pragma unroll
  for (int i = 0; i < BL; ++i) {
    int local;
    const int sg = segment_of(seg, min(r0 + row8 + kRowStep * i, rows - 1), &local);
    const size_t off = (size_t)local * cols + 8 * p8;
    gb[0][i] = segment_w(seg, sg) + off;
    if (kMode == kBGate) gb[kMats - 1][i] = w2 + off;
  }
  const int nstage = (cols + kGBK - 1) / kGBK;
  // fetch and store run unconditionally (a step past the end reloads the
  // last one into a buffer nobody reads), so the loads in flight at each
  // store are the same on every path and the wait before it can leave the
  // newer set outstanding
  auto fetch = [&](int s, St& v) {
    const int k0 = min(s, nstage - 1) * kGBK;
#pragma unroll
    for (int i = 0; i < AL; ++i) v.a[i] = *reinterpret_cast<const u32x4*>(ga[i] + k0);
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int i = 0; i < BL; ++i) v.b[mi][i] = *reinterpret_cast<const u32x4*>(gb[mi][i] + k0);
  };
  auto store = [&](int s, const St& v) {
    const int buf = s % kGBufs;
#pragma unroll
    for (int i = 0; i < AL; ++i) sa[buf][slot0 + kRowStep * kGPieces * i] = v.a[i];
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int i = 0; i < BL; ++i) sb[buf][mi][slot0 + kRowStep * kGPieces * i] = v.b[mi][i];
  };
  f32x16_t acc[kParts][kMats][2];
#pragma unroll
  for (int p = 0; p < kParts; ++p)
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi) acc[p][mi][0] = acc[p][mi][1] = f32x16_t{};
  const int arow = 32 * wave + (lane & 31), half = lane >> 5;
  const bool active = tb + 32 * wave < n;  // uniform per wave
  // one step: all of its fragments first, then the MFMAs (step k of the
  // stage into part k % kParts)
  auto compute = [&](int s) {
    const int buf = s % kGBufs;
    if (!active) return;
    u32x4 av[kGBK / 16], bv[kGBK / 16][kMats][2];
#pragma unroll
    for (int k = 0; k < kGBK / 16; ++k) {
      const int piece = 2 * k + half;
      av[k] = sa[buf][gemm_slot(arow, piece)];
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) bv[k][mi][h] = sb[buf][mi][gemm_slot(32 * h + (lane & 31), piece)];
    }
#pragma unroll
    for (int k = 0; k < kGBK / 16; ++k)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[k % kParts][mi][h] = mfma32(av[k], bv[k][mi][h], acc[k % kParts][mi][h]);
  };
  St X, Y;  // register sets: stage s + 1 in flight in one while stage s + 2 is issued into the other
  fetch(0, X);
  fetch(1, Y);
  store(0, X);
  __syncthreads();
  for (int s = 0; s < nstage; s += 2) {  // nstage is even
    fetch(s + 2, X);
    compute(s);
    store(s + 1, Y);  // buffer (s + 1) % 3 was last read at step s - 2
    __syncthreads();
    fetch(s + 3, Y);
    compute(s + 1);
    store(s + 2, X);
    __syncthreads();
  }
  if (!active) return;
#pragma unroll
  for (int span = 1; span < kParts; span *= 2)
#pragma unroll
    for (int p = 0; p + span < kParts; p += 2 * span)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < 2; ++h) acc[p][mi][h] += acc[p + span][mi][h];
  const int t0 = tb + 32 * wave;
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int row = r0 + 32 * h + (lane & 31);
    if (row >= rows) continue;
    int local;
    const int sg = segment_of(seg, row, &local);
    uint16_t* out = segment_out(seg, sg);
    const int srows = sg == 0 ? seg.rows[0] : sg == 1 ? seg.rows[1] : sg == 2 ? seg.rows[2] : seg.rows[3];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int t = t0 + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
      if (t >= n) continue;
      const size_t o = (size_t)t * srows + local;
      const float v = acc[0][0][h][rr];
      uint16_t y;
      if (kMode == kBPlain) y = f2bf(v);
      else if (kMode == kBResidual) y = bf_add(f2bf(v), res[o]);
      else y = bf_mul(f2bf(silu(rbf(v))), f2bf(acc[0][kMats - 1][h][rr]));
      out[o] = y;
    }
  }
}

// ------------------------------------------------- batched decode (skinny)
//
// The weight-shared batched decode step's products on MFMA (a session
// option, like the prefill components): at most 32 tokens per tile, so the
// work is a weight stream. Block = 32 kT weight rows (kT MFMA tiles sharing
// each activation fragment: two for the vocabulary head) x a 32-token tile x
// one of `kb` column ranges;
// wave w of the block sums a quarter of that range into one accumulator per
// tile (k permuted inside each 64-column batch; the weight rows are loaded as
// whole lines and handed to the MFMA operands through LDS), with two batches
// of four k steps in flight (loads are unconditional:
// a batch past the end reloads the last one, so every wait leaves the newer
// batch outstanding). The four wave partials are added as a tree through LDS
// ((w0 + w1) + (w2 + w3)). With kb > 1 (launches with few row tiles: more
// blocks keep every CU streaming) each block stores its partial tile and
// k_mskinny_finish adds the kb partials in column-range order before the
// epilogue; the kernel boundary orders them, so no device-scope fence (an
// L2 write-back on a multi-XCD part) is needed. cols % (512 kb) == 0.
constexpr int kSkSplit = 4;  // waves per block
constexpr int kSkBatch = 4;  // k steps per load batch
enum { kSArgmax = 3 };       // mode: vocabulary head, bf16 logits and each token's (value, first index) max

// The epilogue of a 32 kT-row x 32-token tile held by one wave (tile tx, ty).
template <int kMode, int kMats, int kT>
__device__ __forceinline__ void skinny_epilogue(const f32x16_t (&acc)[kMats][kT], int tx, int ty, int n,
                                                const Segments& seg, const uint16_t* __restrict__ res,
                                                unsigned long long* __restrict__ best) {
  const int lane = threadIdx.x & 63;
  const int rows = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int r0 = tx * 32 * kT, t0 = ty * 32;
#pragma unroll
  for (int h = 0; h < kT; ++h) {
    const int row = r0 + 32 * h + (lane & 31);
    int lr;
    const int os = segment_of(seg, min(row, rows - 1), &lr);
    uint16_t* out = segment_out(seg, os);
    const int srows = os == 0 ? seg.rows[0] : os == 1 ? seg.rows[1] : os == 2 ? seg.rows[2] : seg.rows[3];
#pragma unroll
    for (int rr = 0; rr < 16; ++rr) {
      const int t = t0 + 8 * (rr >> 2) + 4 * (lane >> 5) + (rr & 3);
      const bool ok = t < n && row < rows;
      const size_t o = (size_t)t * srows + lr;
      const float v = acc[0][h][rr];
      uint16_t y = 0;
      if (ok) {
        if (kMode == kBPlain || kMode == kSArgmax) y = f2bf(v);
        else if (kMode == kBResidual) y = bf_add(f2bf(v), res[o]);
        else y = bf_mul(f2bf(silu(rbf(v))), f2bf(acc[kMats - 1][h][rr]));
        out[o] = y;
      }
      if (kMode == kSArgmax) {
        // this token's (value, first index) maximum over the 32 rows of the
        // tile (lanes of one half), kept per tile: best[(tx kT + h) 32 + t
        // mod 32] for k_argmax_tiles (atomics from thousands of tiles on the
        // same few words would serialise)
        unsigned long long key = ok ? logit_key(y, (uint32_t)row) : 0ull;
#pragma unroll
        for (int d = 16; d >= 1; d >>= 1) {
          const unsigned long long o2 = __shfl_xor(key, d, 64);
          key = o2 > key ? o2 : key;
        }
        if ((lane & 31) == 0) best[(size_t)((ty * gridDim.x + tx) * kT + h) * 32 + (t - t0)] = key;
      }
    }
  }
}

template <int kMode, int kT>
__global__ __launch_bounds__(64 * kSkSplit) void k_mskinny(const uint16_t* __restrict__ x, int n, int cols,
                                                           Segments seg, const uint16_t* __restrict__ w2,
                                                           const uint16_t* __restrict__ res,
                                                           unsigned long long* __restrict__ best,
                                                           f32x16_t* __restrict__ part) {
  constexpr int kMats = kMode == kBGate ? 2 : 1;
  __shared__ f32x16_t red[kSkSplit - 1][kMats][kT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int kb = gridDim.z;
  const int rows = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int r0 = blockIdx.x * 32 * kT, t0 = blockIdx.y * 32;
  // a batch of four k steps covers 64 columns: lane half h holds columns
  // [32 h, 32 h + 32) of it, 8 per step, in both operands (the same
  // permutation of k), so each lane reads 64 contiguous bytes of its token
  // row
  const int kq = 32 * (lane >> 5);
  const int span = cols / (kSkSplit * kb), c0 = (blockIdx.z * kSkSplit + wave) * span;
  const uint16_t* xa = x + (size_t)min(t0 + (lane & 31), n - 1) * cols + c0 + kq;
  const int steps = span / 16;  // a multiple of 2 kSkBatch
  f32x16_t acc[kMats][kT];
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
    for (int h = 0; h < kT; ++h) acc[mi][h] = f32x16_t{};
  // Weight rows through LDS: load instruction g gives lane i the 16-byte
  // chunk i & 7 of tile row 8 g + (i >> 3) in the 64-column batch (eight
  // whole 128-byte lines per instruction), stored in this wave's slot with
  // chunk c of row r at position c ^ (r & 7); the MFMA operand of lane l
  // (row 32 h + (l & 31), chunk 4 (l >> 5) + j: the permuted k above) is
  // then read back, the 32 rows of one chunk spread over all banks. Same
  // operands, same products and sums as reading them directly.
  constexpr int G = 4 * kT;  // load instructions per matrix and batch
  __shared__ __align__(16) u32x4 wst[kSkSplit][kMats][32 * kT * 8];
  const int cr = lane >> 3, cc = lane & 7;
  const uint16_t* wrow[kMats][G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    int local;
    const int sg = segment_of(seg, min(r0 + 8 * g + cr, rows - 1), &local);
    wrow[0][g] = segment_w(seg, sg) + (size_t)local * cols + c0 + 8 * cc;
    if (kMode == kBGate) wrow[kMats - 1][g] = w2 + (size_t)local * cols + c0 + 8 * cc;
  }
  struct Set {
    u32x4 a[kSkBatch], b[kMats][G];
  };
  auto load = [&](int s, Set& v) {
    const int k = 16 * min(s, steps - kSkBatch);
#pragma unroll
    for (int j = 0; j < kSkBatch; ++j) v.a[j] = *reinterpret_cast<const u32x4*>(xa + k + 8 * j);
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int g = 0; g < G; ++g) v.b[mi][g] = *reinterpret_cast<const u32x4*>(wrow[mi][g] + k);
  };
  auto mult = [&](const Set& v) {
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int g = 0; g < G; ++g) wst[wave][mi][(8 * g + cr) * 8 + (cc ^ cr)] = v.b[mi][g];
#pragma unroll
    for (int j = 0; j < kSkBatch; ++j)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
        for (int h = 0; h < kT; ++h) {
          const int r = 32 * h + (lane & 31);
          const u32x4 bq = wst[wave][mi][r * 8 + ((4 * (lane >> 5) + j) ^ (lane & 7))];
          acc[mi][h] = mfma32(v.a[j], bq, acc[mi][h]);
        }
  };
  Set P, Q;
  load(0, P);
  for (int s = 0; s < steps; s += 2 * kSkBatch) {
    load(s + kSkBatch, Q);
    mult(P);
    load(s + 2 * kSkBatch, P);
    mult(Q);
  }
  if (wave > 0) {
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int h = 0; h < kT; ++h) red[wave - 1][mi][h][lane] = acc[mi][h];
  }
  __syncthreads();
  if (wave > 0) return;
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
    for (int h = 0; h < kT; ++h)
      acc[mi][h] = (acc[mi][h] + red[0][mi][h][lane]) + (red[1][mi][h][lane] + red[2][mi][h][lane]);
  if (kb == 1) {
    skinny_epilogue<kMode, kMats, kT>(acc, blockIdx.x, blockIdx.y, n, seg, res, best);
    return;
  }
  const size_t tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
  f32x16_t* mine = part + (((size_t)blockIdx.z * gridDim.y * gridDim.x + tile) * kMats * kT) * 64;
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
    for (int h = 0; h < kT; ++h) mine[(mi * kT + h) * 64 + lane] = acc[mi][h];
}

// Each token's (value, first index) maximum over the per-tile maxima of a
// kSArgmax launch (tiles x 32 keys per token tile; 0 = no candidate): one
// block per token.
__global__ __launch_bounds__(256) void k_argmax_tiles(const unsigned long long* __restrict__ keys, int tiles,
                                                      int n, unsigned long long* __restrict__ best) {
  __shared__ unsigned long long wmax[4];
  const int t = blockIdx.x, tt = t / 32;
  unsigned long long m = 0ull;
  for (int i = threadIdx.x; i < tiles; i += blockDim.x) {
    const unsigned long long k = keys[((size_t)tt * tiles + i) * 32 + (t & 31)];
    m = k > m ? k : m;
  }
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) {
    const unsigned long long o = __shfl_xor(m, d, 64);
    m = o > m ? o : m;
  }
  if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
  __syncthreads();
  if (threadIdx.x == 0 && t < n) {
    for (int i = 1; i < 4; ++i) m = wmax[i] > m ? wmax[i] : m;
    best[t] = m;
  }
}

// The kb column-range partials of each tile of a split k_mskinny launch,
// added in range order, then the epilogue: one wave per (row tile, token
// tile), all of its partials requested before the first add.
template <int kMode, int kT>
__global__ __launch_bounds__(64) void k_mskinny_finish(const f32x16_t* __restrict__ part, int kb, int n,
                                                       Segments seg, const uint16_t* __restrict__ res,
                                                       unsigned long long* __restrict__ best) {
  constexpr int kMats = kMode == kBGate ? 2 : 1, kMaxKb = 8;
  const int lane = threadIdx.x;
  const size_t tiles = (size_t)gridDim.y * gridDim.x, tile = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
  f32x16_t acc[kMats][kT];
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
    for (int h = 0; h < kT; ++h) {
      f32x16_t v[kMaxKb];
#pragma unroll
      for (int z = 0; z < kMaxKb; ++z)
        if (z < kb) v[z] = part[(((size_t)z * tiles + tile) * kMats * kT + mi * kT + h) * 64 + lane];
      acc[mi][h] = v[0];
#pragma unroll
      for (int z = 1; z < kMaxKb; ++z)
        if (z < kb) acc[mi][h] = acc[mi][h] + v[z];
    }
  skinny_epilogue<kMode, kMats, kT>(acc, blockIdx.x, blockIdx.y, n, seg, res, best);
}

// ---------------------------------------------------------------- experts
//
// Grouped expert projections (the reference's grouped routed/shared expert
// stages, qwen35_wmma_moe.hex): the chunk's (token, slot) assignments are
// bucketed by expert, every expert's weights are streamed once per chunk
// and applied to all of its tokens, the shared expert runs as a dense
// product over all tokens, and the routed down products are summed per
// token over the slots in slot order before the reference's epilogue.

// One wave's 32 x 32 MFMA tile over k in [0, cols): A rows at xa, B rows at
// w[mi] (both already offset by the lane's row and k quarter). kParts partial
// sums over rotating k steps, added as a tree.
template <int kParts, int kMats>
__device__ __forceinline__ void mfma_tile(const uint16_t* xa, const uint16_t* const (&w)[kMats], int cols,
                                          f32x16_t (&out)[kMats]) {
  f32x16_t acc[kParts][kMats];
#pragma unroll
  for (int p = 0; p < kParts; ++p)
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi) acc[p][mi] = f32x16_t{};
  const int steps = cols / 16;
  int st = 0;
  for (; st + kParts <= steps; st += kParts) {
    u32x4 a[kParts], b[kParts][kMats];
#pragma unroll
    for (int p = 0; p < kParts; ++p) {
      a[p] = *reinterpret_cast<const u32x4*>(xa + 16 * (st + p));
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi) b[p][mi] = *reinterpret_cast<const u32x4*>(w[mi] + 16 * (st + p));
    }
#pragma unroll
    for (int p = 0; p < kParts; ++p)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi) acc[p][mi] = mfma32(a[p], b[p][mi], acc[p][mi]);
  }
  for (int p = 0; st < steps; ++st, ++p) {
    const u32x4 a = *reinterpret_cast<const u32x4*>(xa + 16 * st);
#pragma unroll
    for (int q = 0; q < kParts; ++q) {
      if (q != p) continue;
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi)
        acc[q][mi] = mfma32(a, *reinterpret_cast<const u32x4*>(w[mi] + 16 * st), acc[q][mi]);
    }
  }
#pragma unroll
  for (int span = 1; span < kParts; span *= 2)
#pragma unroll
    for (int p = 0; p + span < kParts; p += 2 * span)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi) acc[p][mi] += acc[p + span][mi];
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi) out[mi] = acc[0][mi];
}

// mfma_tile with the weight rows loaded as whole 128-byte lines: for each
// 64-column batch (four k steps), load instruction g gives lane i the
// 16-byte chunk i & 7 of tile row 8 g + (i >> 3) (wl[mi][g]: that row's
// chunk at column 0), stored in the wave's LDS slot st[mi] with chunk c of
// row r at position c ^ (r & 7); the B operand of lane l for step p (row
// l & 31, columns 16 p + 8 (l >> 5): chunk 2 p + (l >> 5)) is read back. The
// steps go to the same rotating partial sums in the same order, so the
// results equal mfma_tile's. cols % 64 == 0, kParts divides 4.
template <int kParts, int kMats>
__device__ __forceinline__ void mfma_tile_lines(const uint16_t* xa, const uint16_t* const (&wl)[kMats][4], int cols,
                                                u32x4 (*st)[32 * 8], f32x16_t (&out)[kMats]) {
  static_assert(4 % kParts == 0, "parts per batch");
  const int lane = threadIdx.x & 63, cr = lane >> 3, cc = lane & 7, r = lane & 31, h = lane >> 5;
  f32x16_t acc[kParts][kMats];
#pragma unroll
  for (int p = 0; p < kParts; ++p)
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi) acc[p][mi] = f32x16_t{};
  struct Set {
    u32x4 a[4], b[kMats][4];
  };
  const int batches = cols / 64;
  auto load = [&](int bt, Set& v) {
    const int k = 64 * min(bt, batches - 1);
#pragma unroll
    for (int p = 0; p < 4; ++p) v.a[p] = *reinterpret_cast<const u32x4*>(xa + k + 16 * p);
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int g = 0; g < 4; ++g) v.b[mi][g] = *reinterpret_cast<const u32x4*>(wl[mi][g] + k);
  };
  auto mult = [&](const Set& v) {
#pragma unroll
    for (int mi = 0; mi < kMats; ++mi)
#pragma unroll
      for (int g = 0; g < 4; ++g) st[mi][(8 * g + cr) * 8 + (cc ^ cr)] = v.b[mi][g];
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi) {
        const u32x4 bq = st[mi][r * 8 + ((2 * p + h) ^ (r & 7))];
        acc[p % kParts][mi] = mfma32(v.a[p], bq, acc[p % kParts][mi]);
      }
  };
  // two batches in flight (loads past the end repeat the last batch, which
  // is not multiplied)
  Set P, Q;
  load(0, P);
  for (int bt = 0; bt < batches; bt += 2) {
    load(bt + 1, Q);
    mult(P);
    load(bt + 2, P);
    if (bt + 1 < batches) mult(Q);  // uniform
  }
#pragma unroll
  for (int span = 1; span < kParts; span *= 2)
#pragma unroll
    for (int p = 0; p + span < kParts; p += 2 * span)
#pragma unroll
      for (int mi = 0; mi < kMats; ++mi) acc[p][mi] += acc[p + span][mi];
#pragma unroll
  for (int mi = 0; mi < kMats; ++mi) out[mi] = acc[0][mi];
}

// Buckets: eoff[e] .. eoff[e + 1] index order[], which holds assignment
// indices t * top_k + slot. The order inside a bucket is whatever the
// atomics give: each MFMA output element is its own dot product, unaffected
// by the rows it shares a tile with, so results do not depend on it.
__global__ __launch_bounds__(1024) void k_moe_bucket(const int* __restrict__ ids, int assignments, int experts,
                                                     int* __restrict__ eoff, int* __restrict__ order) {
  extern __shared__ int bucket_lds[];
  int* cnt = bucket_lds;
  int* cur = bucket_lds + experts;
  for (int e = threadIdx.x; e < experts; e += blockDim.x) cnt[e] = 0;
  __syncthreads();
  for (int a = threadIdx.x; a < assignments; a += blockDim.x) atomicAdd(&cnt[ids[a]], 1);
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < experts; ++e) {
      cur[e] = run;
      eoff[e] = run;
      run += cnt[e];
    }
    eoff[experts] = run;
  }
  __syncthreads();
  for (int a = threadIdx.x; a < assignments; a += blockDim.x) order[atomicAdd(&cur[ids[a]], 1)] = a;
}

constexpr int kXWaves = 4;                 // waves per expert block, 32 weight rows each
constexpr int kXRows = 32 * kXWaves;       // weight rows per expert block

// Gate/up of expert blockIdx.y (blockIdx.y == experts: the shared expert over
// all n tokens) for its assignments [32 bz, +32), rows [kXRows bx, +kXRows)
// of width `width`. Epilogues (moe.hex:254-369): routed bf16((silu(bf16 g) * bf16 u) *
// p_slot) into act[t][slot * inter + row]; shared bf16(bf16(bf16(silu(bf16 g))
// * bf16 u) * sigmoid(l_E)) into act[t][top_k * inter + row].
__global__ __launch_bounds__(64 * kXWaves) void k_mmoe_gate(
    const uint16_t* __restrict__ x, int hidden, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ sgate,
    const uint16_t* __restrict__ sup, const int* __restrict__ eoff, const int* __restrict__ order,
    const float* __restrict__ probs, const float* __restrict__ logits, int experts, int top_k,
    int inter, int shared_inter, int n, uint16_t* __restrict__ act) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const bool shared = e == experts;
  const int width = shared ? shared_inter : inter;
  const int begin = shared ? 0 : eoff[e];
  const int count = shared ? n : eoff[e + 1] - begin;
  const int r0 = blockIdx.x * kXRows + 32 * wave;
  if (count == 0 || r0 >= width) return;  // uniform per wave; no barriers below
  const int kq = 8 * (lane >> 5);
  const uint16_t* gbase = shared ? sgate : gate + (size_t)e * inter * hidden;
  const uint16_t* ubase = shared ? sup : up + (size_t)e * inter * hidden;
  const int act_rows = top_k * inter + shared_inter;
  const int row = r0 + (lane & 31);
  {
    const int m0 = 32 * blockIdx.z;
    if (m0 >= count) return;
    const int i = min(m0 + (lane & 31), count - 1);
    const int t = shared ? i : order[begin + i] / top_k;
    f32x16_t acc[2];
    if (hidden % 64 == 0) {  // uniform
      __shared__ __align__(16) u32x4 gst[kXWaves][2][32 * 8];
      const uint16_t* wl[2][4];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const size_t off = (size_t)min(r0 + 8 * g + (lane >> 3), width - 1) * hidden + 8 * (lane & 7);
        wl[0][g] = gbase + off;
        wl[1][g] = ubase + off;
      }
      mfma_tile_lines<2, 2>(x + (size_t)t * hidden + kq, wl, hidden, gst[wave], acc);
    } else {
      const int wrow = min(r0 + (lane & 31), width - 1);
      const uint16_t* w[2] = {gbase + (size_t)wrow * hidden + kq, ubase + (size_t)wrow * hidden + kq};
      mfma_tile<2, 2>(x + (size_t)t * hidden + kq, w, hidden, acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mi = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (mi >= count || row >= width) continue;
      const float gb = rbf(acc[0][r]), ub = rbf(acc[1][r]);
      const float activated = silu(gb);
      if (shared) {
        const float shared_prob = sigmoid(logits[(size_t)mi * (experts + 1) + experts]);
        act[(size_t)mi * act_rows + top_k * inter + row] = f2bf(rbf(rbf(activated) * ub) * shared_prob);
      } else {
        const int a = order[begin + mi];
        const int ta = a / top_k, slot = a - ta * top_k;
        act[(size_t)ta * act_rows + slot * inter + row] = f2bf((activated * ub) * probs[a]);
      }
    }
  }
}

// Down of expert blockIdx.y (== experts: the shared expert) for its
// assignments [32 bz, +32): F32 part[a][o] = sum_i act[t][slot * inter + i] down[e][o][i]
// (shared: spart[t][o] over act[t][top_k * inter + i]), rows o in
// [kXRows bx, +kXRows) of hidden.
__global__ __launch_bounds__(64 * kXWaves) void k_mmoe_down(
    const uint16_t* __restrict__ act, const uint16_t* __restrict__ down,
    const uint16_t* __restrict__ sdown, const int* __restrict__ eoff, const int* __restrict__ order,
    int experts, int top_k, int inter, int shared_inter, int hidden, int n, float* __restrict__ part,
    float* __restrict__ spart) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int e = blockIdx.y;
  const bool shared = e == experts;
  const int width = shared ? shared_inter : inter;  // the product's k extent
  const int begin = shared ? 0 : eoff[e];
  const int count = shared ? n : eoff[e + 1] - begin;
  const int o0 = blockIdx.x * kXRows + 32 * wave;
  if (count == 0 || o0 >= hidden) return;  // uniform per wave; no barriers below
  const int kq = 8 * (lane >> 5);
  const uint16_t* dbase = shared ? sdown : down + (size_t)e * hidden * inter;
  const int act_rows = top_k * inter + shared_inter;
  const int o = o0 + (lane & 31);
  {
    const int m0 = 32 * blockIdx.z;
    if (m0 >= count) return;
    const int i = min(m0 + (lane & 31), count - 1);
    size_t arow;
    if (shared) {
      arow = (size_t)i * act_rows + top_k * inter;
    } else {
      const int a = order[begin + i];
      const int ta = a / top_k;
      arow = (size_t)ta * act_rows + (size_t)(a - ta * top_k) * inter;
    }
    f32x16_t acc[1];
    if (width % 64 == 0) {  // uniform
      __shared__ __align__(16) u32x4 dst_[kXWaves][1][32 * 8];
      const uint16_t* wl[1][4];
#pragma unroll
      for (int g = 0; g < 4; ++g)
        wl[0][g] = dbase + (size_t)min(o0 + 8 * g + (lane >> 3), hidden - 1) * width + 8 * (lane & 7);
      mfma_tile_lines<4, 1>(act + arow + kq, wl, width, dst_[wave], acc);
    } else {
      const uint16_t* w[1] = {dbase + (size_t)min(o0 + (lane & 31), hidden - 1) * width + kq};
      mfma_tile<4, 1>(act + arow + kq, w, width, acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int mi = m0 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
      if (mi >= count || o >= hidden) continue;
      if (shared) spart[(size_t)mi * hidden + o] = acc[0][r];
      else part[(size_t)order[begin + mi] * hidden + o] = acc[0][r];
    }
  }
}

// out[t][o] = bf16(bf16(routed + res) (+) bf16(shared)) with routed summed
// over the slots in slot order (the epilogue of moe.hex:371-471).
__global__ __launch_bounds__(kBlock) void k_moe_combine(const float* __restrict__ part,
                                                        const float* __restrict__ spart,
                                                        const uint16_t* __restrict__ res, int hidden,
                                                        int top_k, uint16_t* __restrict__ out) {
  const int t = blockIdx.y;
  for (int o = blockIdx.x * kBlock + threadIdx.x; o < hidden; o += gridDim.x * kBlock) {
    const float* p = part + (size_t)t * top_k * hidden + o;
    float routed = p[0];
    for (int slot = 1; slot < top_k; ++slot) routed += p[(size_t)slot * hidden];
    const size_t i = (size_t)t * hidden + o;
    out[i] = bf_add(f2bf(routed + bf2f(res[i])), f2bf(spart[i]));
  }
}

// Matrix-core attention of the prompt path: the attention component of the
// reference's matrix-core prefill (CATENA_WMMA_COMPONENTS "attention",
// qwen35.rs:467-503 over qwen35_wmma_attention.hex), with its rounding
// points: the score bf16(q.k * scale) with q.k on the matrix cores and keys
// after the query's position at -inf (score-write, :3-22); probabilities
// bf16(exp(s - max) / den) over the row's maximum and exponential sum
// (softmax.write, :242-258; a masked score contributes 0); the context summed
// on the matrix cores from those BF16 probabilities and written as
// bf16(bf16(ctx) * sigmoid(gate)) (context-write, :503-530). The F32 sums
// inside the products and of the denominator run in orders of their own, the
// exponentials are the hardware's 2^x (about 1 ulp from the reference's exp)
// and a probability is its exponential times the reciprocal of the
// denominator (within 1 ulp of the quotient): F32-level differences under
// the BF16 rounding points, a tolerance-level path as the reference's own
// matrix-core path is.
//
// Block = (query head, 32 consecutive rows of the chunk), kAWaves waves; the
// 32-key tiles up to the last row's position are dealt to the waves round
// robin. Pass 1: each wave forms its tiles' scores S^T = K Q^T (A = the 32
// key rows, B = the 32 query rows, both as 16-byte fragments along the head
// dimension; lane l then holds 16 keys of query l % 32) and keeps a running
// maximum and exponential sum per query; the waves' pairs are merged in wave
// order. Pass 2 recomputes the same scores (same products, same bits), turns
// them into BF16 probabilities, which sit in the registers as the B operand
// of O^T = V^T P^T, and accumulates the context per 32-channel tile. V^T is
// an LDS transpose of the tile's value rows: key pairs packed into 32-bit
// words, positions within each 16 keys with index bits 2 and 3 swapped so
// that a lane's 8 A elements are the 8 keys of its probability registers.
// The waves' context partials are added in wave order through LDS.
constexpr int kAWaves = 4;
constexpr int kAVWords = 18;  // words per transposed value row: 16 key pairs + 2 (72 B, conflict-free stores)

// e^x through the hardware's 2^x (v_exp_f32, about 1 ulp; 2^-inf = 0): the
// probabilities' exponentials of the matrix-core attention only.
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504f); }

template <int HD>
__global__ __launch_bounds__(64 * kAWaves) void k_mattention(
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ qg, const uint16_t* __restrict__ cache,
    int64_t key_base, int64_t value_base, const uint64_t* __restrict__ params, int t, int rows_n, int kvs,
    int heads, int heads_per_kv, float scale, uint16_t* __restrict__ out) {
  static_assert(HD % 64 == 0 && HD <= 256, "head dims of whole 64-channel pairs of tiles");
  constexpr int KS = HD / 16;  // k steps of a score product
  constexpr int CT = HD / 32;  // 32-channel tiles of the context
  constexpr int PU = HD / 32;  // (key pair, 8-channel group) units of a value tile per lane
  __shared__ __align__(16) uint32_t vt[kAWaves][HD][kAVWords];
  __shared__ float mstat[kAWaves][32], dstat[kAWaves][32];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int c = lane & 31, h = lane >> 5;
  const int head = blockIdx.x, r0 = blockIdx.y * 32;
  const int64_t qs = (int64_t)heads * HD;
  const int row = min(r0 + c, rows_n - 1);
  const int64_t pos = step_position(params, t + row);
  const int64_t last = step_position(params, t + min(r0 + 31, rows_n - 1));
  const int tiles = (int)(last >> 5) + 1;
  const int64_t kvoff = (int64_t)(head / heads_per_kv) * HD;
  const float ninf = bitsf(0xff800000u);
  u32x4 qf[KS];
  {
    const uint16_t* qr = q + row * qs + head * HD + 8 * h;
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const u32x4*>(qr + 16 * s);
  }
  // key rows past the last row's position read that position's row (masked)
  const uint16_t* kb = cache + key_base + kvoff + 8 * h;
  u32x4 kf[KS];
  auto load_keys = [&](int j) {
    const uint16_t* kr = kb + min((int64_t)32 * j + c, last) * kvs;
#pragma unroll
    for (int s = 0; s < KS; ++s) kf[s] = *reinterpret_cast<const u32x4*>(kr + 16 * s);
  };
  // register r: key 32 j + 8 (r / 4) + 4 h + r % 4 of query row r0 + c
  auto scores = [&](int j, f32x16_t& sc) {
    f32x16_t acc = {};
#pragma unroll
    for (int s = 0; s < KS; ++s) acc = mfma32(kf[s], qf[s], acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int64_t key = 32 * (int64_t)j + 8 * (r >> 2) + 4 * h + (r & 3);
      sc[r] = key <= pos ? rbf(acc[r] * scale) : ninf;
    }
  };
  // pass 1: running maximum and exponential sum per query
  float m = ninf, den = 0.0f;
  if (wave < tiles) load_keys(wave);
#pragma unroll 1
  for (int j = wave; j < tiles; j += kAWaves) {
    f32x16_t sc;
    scores(j, sc);
    if (j + kAWaves < tiles) load_keys(j + kAWaves);
    float tm = sc[0];
#pragma unroll
    for (int r = 1; r < 16; ++r) tm = fmaxf(tm, sc[r]);
    tm = fmaxf(tm, __shfl_xor(tm, 32, 64));
    const float mn = fmaxf(m, tm);
    float e = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) e += sc[r] == ninf ? 0.0f : fast_exp(sc[r] - mn);
    e += __shfl_xor(e, 32, 64);  // the same sum in both halves (addition commutes)
    den = (m == ninf ? 0.0f : den * fast_exp(m - mn)) + e;
    m = mn;
  }
  if (h == 0) {
    mstat[wave][c] = m;
    dstat[wave][c] = den;
  }
  __syncthreads();
  float M = mstat[0][c];
#pragma unroll
  for (int w = 1; w < kAWaves; ++w) M = fmaxf(M, mstat[w][c]);
  float D = 0.0f;
#pragma unroll
  for (int w = 0; w < kAWaves; ++w)
    if (mstat[w][c] != ninf) D += dstat[w][c] * fast_exp(mstat[w][c] - M);
  const float rD = 1.0f / D;
  // pass 2: probabilities and the context
  uint32_t* vw = &vt[wave][0][0];
  const uint16_t* vb = cache + value_base + kvoff;
  u32x4 vv[PU][2];
  auto load_values = [&](int j) {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int pu = lane + 64 * u, kp = pu & 15, cg = pu >> 4;
      const int64_t k0 = 32 * (int64_t)j + 2 * kp;
      vv[u][0] = *reinterpret_cast<const u32x4*>(vb + min(k0, last) * kvs + 8 * cg);
      vv[u][1] = *reinterpret_cast<const u32x4*>(vb + min(k0 + 1, last) * kvs + 8 * cg);
    }
  };
  auto store_values = [&]() {
#pragma unroll
    for (int u = 0; u < PU; ++u) {
      const int pu = lane + 64 * u, kp = pu & 15, cg = pu >> 4;
      const int k = 2 * kp;
      const int p = (k & ~12) | ((k & 4) << 1) | ((k & 8) >> 1);  // bits 2 and 3 swapped
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t a = vv[u][0][i >> 1], b = vv[u][1][i >> 1];
        const uint32_t lo = (i & 1) ? a >> 16 : a & 0xffffu;
        const uint32_t hi = (i & 1) ? b & 0xffff0000u : b << 16;
        vw[(8 * cg + i) * kAVWords + (p >> 1)] = lo | hi;
      }
    }
  };
  f32x16_t o[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) o[ct] = f32x16_t{};
  if (wave < tiles) {
    load_keys(wave);
    load_values(wave);
  }
#pragma unroll 1
  for (int j = wave; j < tiles; j += kAWaves) {
    f32x16_t sc;
    scores(j, sc);
    const bool more = j + kAWaves < tiles;
    if (more) load_keys(j + kAWaves);
    u32x4 pb[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int r = 8 * ks + 2 * i;
        const uint32_t p0 = sc[r] == ninf ? 0u : f2bf(fast_exp(sc[r] - M) * rD);
        const uint32_t p1 = sc[r + 1] == ninf ? 0u : f2bf(fast_exp(sc[r + 1] - M) * rD);
        pb[ks][i] = p0 | (p1 << 16);
      }
    store_values();
    if (more) load_values(j + kAWaves);
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const uint32_t* src = vw + (32 * ct + c) * kAVWords + 8 * ks + 4 * h;
        const uint2 x0 = *reinterpret_cast<const uint2*>(src), x1 = *reinterpret_cast<const uint2*>(src + 2);
        const u32x4 a = {x0.x, x0.y, x1.x, x1.y};
        o[ct] = mfma32(a, pb[ks], o[ct]);
      }
    __builtin_amdgcn_wave_barrier();
  }
  // waves' partials added in wave order, one half of the channel tiles at a
  // time (every wave's partials of a half fit the value tiles' LDS); wave w
  // finishes tiles w, w + kAWaves, ... of the half. The half is a compile-time
  // constant so that the accumulators stay in registers.
  __syncthreads();
  float* red = reinterpret_cast<float*>(&vt[0][0][0]);
  constexpr int HT = CT / 2;
  static_assert(kAWaves * HT * 16 * 64 * 4 <= (int)sizeof(vt), "partials fit the value tiles");
  const int rr = r0 + c;
  auto finish = [&](auto half_c) {
    constexpr int half = decltype(half_c)::value;
#pragma unroll
    for (int i = 0; i < HT; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) red[((wave * HT + i) * 16 + r) * 64 + lane] = o[half * HT + i][r];
    __syncthreads();
    if (rr < rows_n) {
      const uint16_t* gate = qg + (int64_t)rr * 2 * qs + (int64_t)head * 2 * HD + HD;
      uint16_t* dst = out + (int64_t)rr * qs + (int64_t)head * HD;
      for (int i = wave; i < HT; i += kAWaves) {
        const int ct = half * HT + i;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int ch = 32 * ct + 8 * g + 4 * h;
          const uint2 gv = *reinterpret_cast<const uint2*>(gate + ch);
          uint32_t packed[2];
#pragma unroll
          for (int e = 0; e < 4; e += 2) {
            uint32_t two = 0;
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              const int r = 4 * g + e + x;
              float v = red[(i * 16 + r) * 64 + lane];
#pragma unroll
              for (int w = 1; w < kAWaves; ++w) v += red[((w * HT + i) * 16 + r) * 64 + lane];
              const uint32_t gw = e == 0 ? gv.x : gv.y;
              const float gs = sigmoid(bf2f((uint16_t)(x ? gw >> 16 : gw & 0xffffu)));
              two |= (uint32_t)f2bf(rbf(v) * gs) << (16 * x);
            }
            packed[e >> 1] = two;
          }
          *reinterpret_cast<uint2*>(dst + ch) = make_uint2(packed[0], packed[1]);
        }
      }
    }
    __syncthreads();
  };
  finish(std::integral_constant<int, 0>{});
  finish(std::integral_constant<int, 1>{});
}

}  // namespace cq35
