// Weight-shared decode step for MoE sessions (same model and capacity, one
// token each): the non-expert weights of every layer are read once for all
// the sessions' tokens, the routed experts once per distinct expert of the
// round (the union of the sessions' top-k), the shared expert once.
//
// The reference steps sessions one after another (src/server/engine.rs:
// 143-207); each token's arithmetic here is exactly its single-session
// decode step (the per-kernel kernels of gemv.h / attention.h and the
// persistent step, bit for bit):
//
//  k_ws256     S256 grouped projections (qwen35.group-project) for NB tokens
//              staged in LDS, k_project256's lane order and tree;
//  k_broute   the post-mixer norm and the F32 router rows (moe.hex:4-84),
//              every token per block, k_router_select's lane order and tree;
//  k_sselect   per token (one wave each): stable rank top-k and the softmax
//              weights (moe.hex:86-252), the ids also copied to the session's
//              export row, each (token, slot) appended to its expert's list;
//  k_bgate     per distinct selected expert its gate/up rows applied to every
//              token that selected it, with that token's weight; the shared
//              expert's rows applied to every token (moe.hex:254-333);
//  k_bdown     per (output row, token): the S32 over the token's concatenated
//              expert rows in slot order, the shared S32 and the residual
//              (moe.hex:371-434); the rows of experts that several tokens
//              chose are read from HBM once and from L2 after;
//  k_bscores / decode attention per session over its own cache: the scores
//  k_bflash /  (k_attn_scores' order), then split-K ranges (one block per
//  k_bmerge    (KV head, range), all the group's query heads, one channel
//              per thread) merged in ascending order, or the single chain per
//              query head, as the session's split threshold selects;
//              k_attn_values' arithmetic.
#pragma once

#include "attention.h"
#include "batch.h"

namespace cq35 {

// Pointers taken from the session table are generic; loads through them are
// made global (not flat) so that the wait counters track them alone.
template <typename T>
__device__ __forceinline__ const __attribute__((address_space(1))) T* gmem(const T* p) {
  return (const __attribute__((address_space(1))) T*)p;
}

// ------------------------------------------------ S256 grouped projection

// Rows of up to four segments for NB tokens of already normalised rows
// (cols <= kBatchChunk, staged once as F32): token t's output row r of
// segment s goes to seg.out[s][t * seg.rows[s] + r]. Each wave runs kRW rows,
// one at a time, 64 lanes per row, lane l visiting quads l, l + 64, ... in
// order.
template <int kRW, int NB>
__global__ __launch_bounds__(kBlock) void k_ws256(const uint16_t* __restrict__ x, int tokens, int groups,
                                                  Segments seg, int cols) {
  constexpr int RW = kRW, NQ = 4;
  extern __shared__ __align__(16) float xf[];  // [NB][cols]
  int rb, tg;
  batch_block(blockIdx.x, groups, &rb, &tg);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quads = cols >> 3;
  const int total = seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
  const int row0 = (rb * 4 + wave) * RW;
  const int t0 = tg * NB;
  u32x4 wv[RW][NQ];
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    int local;
    const int s = segment_of(seg, min(row0 + r, total - 1), &local);
    const uint16_t* wr = segment_w(seg, s) + (size_t)local * cols;
#pragma unroll
    for (int j = 0; j < NQ; ++j) wv[r][j] = ldq(wr, min(lane + 64 * j, quads - 1));
  }
  stage_f32<NB>(xf, x, tokens, t0, cols, 0, cols);
#pragma unroll
  for (int r = 0; r < RW; ++r) {
    Quad acc[NB];
#pragma unroll
    for (int t = 0; t < NB; ++t) quad_zero(acc[t]);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (lane + 64 * j < quads) {
#pragma unroll
        for (int t = 0; t < NB; ++t) quad_acc_staged(acc[t], xf + t * cols, quads, lane + 64 * j, wv[r][j]);
      }
    const int row = row0 + r;
    int local;
    const int s = segment_of(seg, min(row, total - 1), &local);
    const int srows = s == 0 ? seg.rows[0] : s == 1 ? seg.rows[1] : s == 2 ? seg.rows[2] : seg.rows[3];
    static_assert(NB % 2 == 0, "token trees in pairs");
#pragma unroll
    for (int t = 0; t < NB; t += 2) {
      const float tot = quad_tree64_pair_end(acc[t], acc[t + 1]);  // token t in lane 31, t + 1 in lane 63
      const float v0 = lane_value(tot, 31);
      const float v1 = lane_value(tot, 63);
      if (lane == 0 && row < total) {
        if (t0 + t < tokens) segment_out(seg, s)[(size_t)(t0 + t) * srows + local] = f2bf(v0);
        if (t0 + t + 1 < tokens) segment_out(seg, s)[(size_t)(t0 + t + 1) * srows + local] = f2bf(v1);
      }
    }
  }
}

// ---------------------------------------------------------------- router

// qwen35.normalize of one row by one wave, the same sums as norm_finish's
// block-wide tree: lane l holds octets 4l .. 4l + 3 (xv, with the norm
// weights w0/w1 of those octets), so ((o0 + o1) + (o2 + o3)) is the tree's
// first two cross-thread levels, lane strides 1, 2, 4, 8 its next four (each
// 16 lanes are one of its waves), and strides 16 then 32 its ((w0 + w1) +
// (w2 + w3)). The normalised octets go to xs (LDS) and, with out, to global
// memory. cols <= 2048.
__device__ __forceinline__ void wave_norm_octets(const u32x4 (&xv)[4], const f32x4 (&w0)[4], const f32x4 (&w1)[4],
                                                 int cols, float eps, u32x4* xs, uint16_t* __restrict__ out) {
  const int lane = threadIdx.x & 63, octs = cols >> 3;
  float sq[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) sq[q] = 4 * lane + q < octs ? octet_squares(xv[q]) : 0.0f;
  float t = (sq[0] + sq[1]) + (sq[2] + sq[3]);
  t = t + lane_down<1>(t);
  t = t + lane_down<2>(t);
  t = t + lane_down<4>(t);
  t = t + lane_down<8>(t);
  t = t + lane_down<16>(t);
  t = t + lane_down<32>(t);
  const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, t)));
  const float inverse = 1.0f / nsqrt(sum / (float)cols + eps);
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int o = 4 * lane + q;
    if (o < octs) {
      const u32x4 y = octet_scale(xv[q], inverse, w0[q], w1[q]);
      xs[o] = y;
      if (out) reinterpret_cast<u32x4*>(out)[o] = y;
    }
  }
}

// Post-mixer norm and router logits of every token: rows [0, E) routed, row
// E the shared-expert gate, F32 weights; one wave per row, all tokens per
// block (each row read once). Every block normalises every token's row
// (wave w the tokens w, w + 4, ...; block 0 also writes them to xout for the
// expert kernels) into LDS, then each wave runs its row: physical lane
// l = 2r + h holds reference lane r's low (h = 0) or high (h = 1)
// accumulator over floats l, l + 64, ..., then lo + hi and the halving tree
// (k_router_select's order). logits [tokens][E + 1].
template <int KJ>  // cols / 64
__global__ __launch_bounds__(kBlock) void k_broute(const uint16_t* __restrict__ raw, const float* __restrict__ norm_w,
                                                   float eps, int tokens, const float* __restrict__ w,
                                                   const float* __restrict__ shared_w, int experts,
                                                   uint16_t* __restrict__ xout, float* __restrict__ logits) {
  constexpr int cols = 64 * KJ;
  extern __shared__ __align__(16) u32x4 xsb[];  // [tokens][cols / 8] normalised rows
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int rows = experts + 1;
  const int row = blockIdx.x * 4 + wave;
  const int rc = min(row, rows - 1);
  const float* wr = rc < experts ? w + (size_t)rc * cols : shared_w;
  float wv[KJ];
#pragma unroll
  for (int j = 0; j < KJ; ++j) wv[j] = wr[lane + 64 * j];
  constexpr int quads = cols >> 3;
  // norm weights of this lane's octets, the same for every token
  f32x4 w0[4], w1[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int o = min(4 * lane + q, quads - 1);
    w0[q] = reinterpret_cast<const f32x4*>(norm_w)[2 * o];
    w1[q] = reinterpret_cast<const f32x4*>(norm_w)[2 * o + 1];
  }
  // wave w normalises tokens w, w + 4, ..., two at a time (both rows'
  // loads issued before either sum)
  for (int t = wave; t < tokens; t += 8) {
    const int t2 = min(t + 4, tokens - 1);
    u32x4 xa[4], xb[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int o = min(4 * lane + q, quads - 1);
      xa[q] = ldq(raw + (size_t)t * cols, o);
      xb[q] = ldq(raw + (size_t)t2 * cols, o);
    }
    wave_norm_octets(xa, w0, w1, cols, eps, xsb + (size_t)t * quads, blockIdx.x == 0 ? xout + (size_t)t * cols : nullptr);
    if (t + 4 < tokens)
      wave_norm_octets(xb, w0, w1, cols, eps, xsb + (size_t)t2 * quads,
                       blockIdx.x == 0 ? xout + (size_t)t2 * cols : nullptr);
  }
  __syncthreads();
  for (int t = 0; t < tokens; ++t) {
    const uint16_t* xt = reinterpret_cast<const uint16_t*>(xsb + (size_t)t * quads);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < KJ; ++j) acc += bf2f(xt[lane + 64 * j]) * wv[j];
    float v = acc + lane_down<1>(acc);
    v += lane_down<32>(v);
    v += lane_down<16>(v);
    v += lane_down<8>(v);
    v += lane_down<4>(v);
    v += lane_down<2>(v);
    if (lane == 0 && row < rows) logits[(size_t)t * rows + row] = v;
  }
}

// Orderable image of a router logit: larger logits give larger images, -0
// equals +0, every non-NaN image is at least 0x00800000 (0 marks absent or
// taken).
__device__ __forceinline__ uint32_t route_order(float le) {
  const uint32_t u = le == 0.0f ? 0u : fbits(le);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
template <int S>
__device__ __forceinline__ uint32_t umax_lane(uint32_t v) {
  const uint32_t o = __builtin_bit_cast(uint32_t, lane_down<S>(__builtin_bit_cast(float, v)));
  return o > v ? o : v;
}

// Top-k of one token per wave (moe.hex:86-252): without NaN logits, k rounds
// of a wave-wide maximum of the images (DPP) and the lowest expert index
// holding it (ballots), which is the stable descending rank; with NaNs the
// rank formula rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)} (the
// largest index of a shared rank takes it, an unassigned rank k keeps
// expert k), as k_router_select does. Then
// p_j = exp(l_j - l_0) / den with den summed left to right from 0. The ids
// also go to row `layer` of the session's export buffer, and each
// (token, slot) with its weight to its expert's list for the gate/up
// kernel (in any order: each token's rows are computed on their own; a
// token's slots repeat an expert only when NaN logits made ranks collide,
// so a list holds at most max_tokens * top_k entries); on its first
// selection an expert takes a slot in the round's list of distinct experts
// (count at ecount[experts]). One block of kBlock threads per 4 tokens.
__global__ __launch_bounds__(kBlock) void k_sselect(const float* __restrict__ logits, int tokens, int experts,
                                                    int top_k, int* __restrict__ ids, float* __restrict__ probs,
                                                    const SessionRows* __restrict__ rows, int layer,
                                                    int* __restrict__ ecount, int* __restrict__ elist, int max_tokens,
                                                    int* __restrict__ uexp) {
  constexpr int PER = 8;  // candidates per lane: experts <= 512
  extern __shared__ float lgs[];  // [4][experts]
  __shared__ int sid[4][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int b = blockIdx.x * 4 + wave;
  if (b >= tokens) return;  // wave-uniform; no barrier below
  float* lg = lgs + wave * experts;
  const float* src = logits + (size_t)b * (experts + 1);
  uint32_t ov[PER];
  bool nan = false;
#pragma unroll
  for (int c = 0; c < PER; ++c) {
    const int e = lane + 64 * c;
    ov[c] = 0u;
    if (e < experts) {
      const float le = src[e];
      lg[e] = le;
      nan |= le != le;
      ov[c] = route_order(le);
    }
  }
  if (!__any(nan)) {
    for (int k = 0; k < top_k; ++k) {
      uint32_t best = ov[0];
#pragma unroll
      for (int c = 1; c < PER; ++c) best = ov[c] > best ? ov[c] : best;
      best = umax_lane<32>(best);
      best = umax_lane<16>(best);
      best = umax_lane<8>(best);
      best = umax_lane<4>(best);
      best = umax_lane<2>(best);
      best = umax_lane<1>(best);
      const uint32_t win = __builtin_amdgcn_readfirstlane(best);
      int e = experts;
#pragma unroll
      for (int c = PER - 1; c >= 0; --c) {
        const unsigned long long hit = __ballot(ov[c] == win);
        if (hit) e = 64 * c + __builtin_ctzll(hit);
      }
#pragma unroll
      for (int c = 0; c < PER; ++c)
        if (64 * c + lane == e) ov[c] = 0u;  // taken
      if (lane == 0) sid[wave][k] = e;
    }
  } else {
    // colliding ranks: the largest expert index takes the rank (an LDS
    // maximum), an unassigned rank k keeps expert k
    if (lane < top_k) sid[wave][lane] = -1;
    for (int e = lane; e < experts; e += 64) {
      const float le = lg[e];
      int rank = 0;
      for (int i = 0; i < experts; ++i) {
        const float o = lg[i];
        rank += (o > le) ? 1 : ((i < e && !(le > o)) ? 1 : 0);
      }
      if (rank < top_k) atomicMax(&sid[wave][rank], e);
    }
    if (lane < top_k && sid[wave][lane] < 0) sid[wave][lane] = lane;
  }
  const int e = lane < top_k ? sid[wave][lane] : 0;
  const float lj = lane < top_k ? lg[e] : 0.0f;
  const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, lj)));
  const float ex = lane < top_k ? hexp(lj - l0) : 0.0f;
  float den = 0.0f;
  for (int j = 0; j < top_k; ++j)
    den = den + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), j));
  if (lane < top_k) {
    const float pj = ex / den;
    probs[b * top_k + lane] = pj;
    ids[b * top_k + lane] = e;
    if (rows->ids[b]) rows->ids[b][layer * top_k + lane] = e;
    const int at = atomicAdd(&ecount[e], 1);
    reinterpret_cast<int2*>(elist)[(size_t)e * max_tokens * top_k + at] = int2{(b << 8) | lane, (int)fbits(pj)};
    if (at == 0) uexp[atomicAdd(&ecount[experts], 1)] = e;
  }
}

// Zero n ints (the experts' list counts before a round's selections).
__global__ void k_zero_ints(int* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0;
}

// ----------------------------------------------------------- expert gate/up

constexpr int kGateRowsPerBlock = 4;  // one row pair (gate, up) per wave

// Block (slot, 4 rows): slot 0 is the shared expert (its waves run every
// token, so they start first), slots 1 .. n the round's distinct selected
// experts (in selection order). Each wave is on its own (no LDS, no
// barrier): it reads its expert, then the head of the expert's list of
// (token, slot) entries, issues its row pair's loads (gate and up, 8 KB) and
// the first two entries' normalised rows (L2), and runs the dual S256
// (k_gate_up's order) per entry, the row of the entry after next loaded
// while an entry computes: routed act[t][slot * I + row] =
// bf16(silu(bf16 g) * bf16 u * p_{t,slot}); shared act[t][K * I + row] =
// bf16(bf16(bf16(silu(bf16 g)) * bf16 u) * sigmoid(l_E)). Small waves keep
// many of them resident per CU, which is what keeps HBM busy here. Loads
// past a list's end are clamped inside the list and the token range (their
// rows are loaded, never used).
// x [tokens][cols] normalised rows, cols = 512 NQ (FULL) or below 512 NQ.
template <int NQ, bool FULL>
__global__ __launch_bounds__(kBlock) void k_bgate(
    const uint16_t* __restrict__ x, int tokens, int cols, const uint16_t* __restrict__ gate,
    const uint16_t* __restrict__ up, const uint16_t* __restrict__ sgate, const uint16_t* __restrict__ sup,
    const int* __restrict__ ecount, const int* __restrict__ elist, const int* __restrict__ uexp,
    const float* __restrict__ probs, const float* __restrict__ logits, int experts, int top_k, int inter,
    int shared_inter, int row_blocks, int max_slots, int max_tokens, uint16_t* __restrict__ act) {
  const int sidx = blockIdx.x / row_blocks, rb = blockIdx.x - sidx * row_blocks;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int quads = FULL ? 64 * NQ : cols >> 3;
  const bool shared = sidx == 0;
  const int slot = sidx - 1;
  const int nrows = shared ? shared_inter : inter;
  const int row = rb * kGateRowsPerBlock + wave;
  if (row >= nrows) return;  // wave-uniform
  // the distinct-expert count and this slot's expert in one round trip
  const int n_u = ecount[experts];
  const int e = shared ? 0 : uexp[max(slot, 0)];
  if (!shared && slot >= n_u) return;  // fewer distinct experts this round
  const int cap = max_tokens * top_k;  // entries one list can hold
  const int2* list = reinterpret_cast<const int2*>(elist) + (size_t)e * cap;
  // count and list head first: they return ahead of the rows
  const int n = shared ? tokens : ecount[e];
  int2 head[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int2 v = list[min(i, cap - 1)];
    head[i] = shared ? int2{min(i, tokens - 1) << 8, 0} : v;
  }
  const uint16_t* g = shared ? sgate + (size_t)row * cols : gate + ((size_t)e * inter + row) * cols;
  const uint16_t* u = shared ? sup + (size_t)row * cols : up + ((size_t)e * inter + row) * cols;
  u32x4 gv[NQ], uv[NQ];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const int o = FULL ? lane + 64 * j : min(lane + 64 * j, quads - 1);
    gv[j] = ldq(g, o);
    uv[j] = ldq(u, o);
  }
  // an entry past the list's end holds whatever the buffer held: its token
  // field is clamped into [0, tokens) as an unsigned value
  auto row_of = [&](int2 entry) {
    return x + (size_t)min((unsigned)(entry.x >> 8), (unsigned)(tokens - 1)) * cols;
  };
  auto load_x = [&](u32x4 (&xq)[NQ], const uint16_t* xr) {
#pragma unroll
    for (int j = 0; j < NQ; ++j) xq[j] = ldq(xr, FULL ? lane + 64 * j : min(lane + 64 * j, quads - 1));
  };
  auto entry_at = [&](int i) {
    const int2 v = list[min(i, cap - 1)];
    return shared ? int2{min(i, tokens - 1) << 8, 0} : v;
  };
  const int act_row = top_k * inter + shared_inter;
  auto run = [&](int2 entry, const u32x4(&xq)[NQ]) {
    // the rows stay packed across entries (unpacked per use, not hoisted)
#pragma unroll
    for (int j = 0; j < NQ; ++j) asm volatile("" : "+v"(gv[j]), "+v"(uv[j]));
    const int t = entry.x >> 8, k = entry.x & 255;
    // the gate row's sums, then the up row's (one accumulator set live)
    Quad ga, ua;
    quad_zero(ga);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (FULL || lane + 64 * j < quads) quad_acc(ga, xq[j], gv[j]);
    const float gsum = quad_tree<64>(ga);
    __builtin_amdgcn_sched_barrier(0);
    quad_zero(ua);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (FULL || lane + 64 * j < quads) quad_acc(ua, xq[j], uv[j]);
    const float usum = quad_tree<64>(ua);
    if (lane == 0) {
      const float gb = rbf(gsum), ub = rbf(usum);
      const float activated = silu(gb);
      if (!shared)
        act[(size_t)t * act_row + (size_t)k * inter + row] = f2bf((activated * ub) * bitsf((uint32_t)entry.y));
      else
        act[(size_t)t * act_row + (size_t)top_k * inter + row] =
            f2bf(rbf(rbf(activated) * ub) * sigmoid(logits[(size_t)t * (experts + 1) + experts]));
    }
  };
  // two entries in flight: A holds the even ones, B the odd ones; an
  // entry's successor but one loads while the entry between them computes
  u32x4 xa[NQ], xb[NQ];
  int2 ea = head[0], eb = head[1];
  load_x(xa, row_of(ea));
  load_x(xb, row_of(eb));
  for (int s = 0; s < n; s += 2) {
    run(ea, xa);
    if (s + 2 < n) {
      ea = entry_at(s + 2);
      load_x(xa, row_of(ea));
    }
    if (s + 1 < n) {
      run(eb, xb);
      if (s + 3 < n) {
        eb = entry_at(s + 3);
        load_x(xb, row_of(eb));
      }
    }
  }
}

// ------------------------------------------------------------- expert down

constexpr int kBDownRows = 8;    // output rows per block
constexpr int kBDownTokens = 2;  // tokens per block

// Block (row block, token group): 16 groups of 16 lanes, group g = output
// row row0 + (g & 7) of token t0 + (g >> 3). Lane q of a group runs
// reference lanes 2q and 2q + 1 of the S32: the pair words 32j + 2q and
// 32j + 2q + 1 (one 8-byte read) of the token's concatenated routed row
// (slot order; expert ids[slot]'s row, 8 reads per slot) and of the shared
// row, each reference lane's chain in j order, then the halving tree
// (partners 16, 8, 4, 2 lanes away across lanes, 1 inside the lane) and
// out = bf16(bf16(routed + residual) (+) bf16(shared)) (k_moe_down's
// order). Two slots' rows in flight while one is summed. The group's
// tokens' activations are staged in LDS. Requires inter % 64 == 0,
// inter <= 512 and shared_inter % 64 == 0, shared_inter <= 512.
__device__ __forceinline__ void pair2_acc(float (&lo)[2], float (&hi)[2], uint2 x, uint2 w) {
  lo[0] += lo2f(x.x) * lo2f(w.x);
  hi[0] += hi2f(x.x) * hi2f(w.x);
  lo[1] += lo2f(x.y) * lo2f(w.y);
  hi[1] += hi2f(x.y) * hi2f(w.y);
}
__global__ __launch_bounds__(kBlock) void k_bdown(const uint16_t* __restrict__ act, int tokens,
                                                  const uint16_t* __restrict__ down,
                                                  const uint16_t* __restrict__ sdown, const int* __restrict__ ids,
                                                  const uint16_t* __restrict__ residual, int hidden, int top_k,
                                                  int inter, int shared_inter, uint16_t* __restrict__ out) {
  extern __shared__ __align__(16) u32x4 as[];  // [kBDownTokens][per_row quads]
  __shared__ int sids[kBDownTokens * 16];
  const int iq = inter >> 3, sq = shared_inter >> 3, rq = top_k * iq, per_row = rq + sq;
  const int lane = threadIdx.x & 63, tid = threadIdx.x;
  const int g = tid >> 4, q = lane & 15;
  const int t0 = blockIdx.y * kBDownTokens;
  const int row = blockIdx.x * kBDownRows + (g & (kBDownRows - 1));
  const int ti = g / kBDownRows;
  const int t = t0 + ti;
  const bool live = t < tokens && row < hidden;
  const int rowc = min(row, hidden - 1), tc = min(t, tokens - 1);
  const int ntok = min(kBDownTokens, tokens - t0);
  for (int i = tid; i < ntok * per_row; i += blockDim.x) {
    const int s = i / per_row, o = i - s * per_row;
    as[i] = ldq(act + (size_t)(t0 + s) * per_row * 8, o);
  }
  // the tokens' expert ids before any weight load: a weight address that
  // waited on an id load would wait for every load in flight
  if (tid < ntok * top_k) sids[tid] = ids[(size_t)t0 * top_k + tid];
  float r_lo[2] = {0.0f, 0.0f}, r_hi[2] = {0.0f, 0.0f}, s_lo[2] = {0.0f, 0.0f}, s_hi[2] = {0.0f, 0.0f};
  // the shared row first (its loads overlap the staging): pairs 32j + 2q
  constexpr int NS = 8, NW = 8;  // 8-byte reads per lane per row (<= 512 wide)
  const uint2* sw = reinterpret_cast<const uint2*>(sdown + (size_t)rowc * shared_inter);
  const int sn = shared_inter >> 6, wn = inter >> 6;  // reads per lane
  uint2 swv[NS];
#pragma unroll
  for (int j = 0; j < NS; ++j) swv[j] = sw[min(q + 16 * j, 16 * sn - 1)];
  __syncthreads();
  const uint2* xr = reinterpret_cast<const uint2*>(as + (size_t)ti * per_row);
  const int* tid_ids = sids + (tc - t0) * top_k;
  auto slot_row = [&](int k) {
    return reinterpret_cast<const uint2*>(down + ((size_t)tid_ids[min(k, top_k - 1)] * hidden + rowc) * inter);
  };
  uint2 wa[NW], wb[NW];
  {
    const uint2* wr = slot_row(0);
#pragma unroll
    for (int j = 0; j < NW; ++j) wa[j] = wr[min(q + 16 * j, 16 * wn - 1)];
  }
  for (int k = 0; k < top_k; k += 2) {
    {
      const uint2* wr = slot_row(k + 1);
#pragma unroll
      for (int j = 0; j < NW; ++j) wb[j] = wr[min(q + 16 * j, 16 * wn - 1)];
    }
#pragma unroll
    for (int j = 0; j < NW; ++j)
      if (j < wn) pair2_acc(r_lo, r_hi, xr[k * (iq * 2) + q + 16 * j], wa[j]);
    {
      const uint2* wr = slot_row(k + 2);
#pragma unroll
      for (int j = 0; j < NW; ++j) wa[j] = wr[min(q + 16 * j, 16 * wn - 1)];
    }
    if (k + 1 < top_k) {
#pragma unroll
      for (int j = 0; j < NW; ++j)
        if (j < wn) pair2_acc(r_lo, r_hi, xr[(k + 1) * (iq * 2) + q + 16 * j], wb[j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (j < sn) pair2_acc(s_lo, s_hi, xr[rq * 2 + q + 16 * j], swv[j]);
  // halving tree over the 32 reference lanes (2 per physical lane)
  float r0 = r_lo[0] + r_hi[0], r1 = r_lo[1] + r_hi[1];
  float h0 = s_lo[0] + s_hi[0], h1 = s_lo[1] + s_hi[1];
  r0 += lane_down<8>(r0), r1 += lane_down<8>(r1), h0 += lane_down<8>(h0), h1 += lane_down<8>(h1);
  r0 += lane_down<4>(r0), r1 += lane_down<4>(r1), h0 += lane_down<4>(h0), h1 += lane_down<4>(h1);
  r0 += lane_down<2>(r0), r1 += lane_down<2>(r1), h0 += lane_down<2>(h0), h1 += lane_down<2>(h1);
  r0 += lane_down<1>(r0), r1 += lane_down<1>(r1), h0 += lane_down<1>(h0), h1 += lane_down<1>(h1);
  const float rv = r0 + r1, sv = h0 + h1;
  if (q == 0 && live) {
    const size_t o = (size_t)t * hidden + row;
    out[o] = bf_add(f2bf(rv + bf2f(residual[o])), f2bf(sv));
  }
}

inline size_t bdown_lds_bytes(int per_row_quads) { return (size_t)kBDownTokens * per_row_quads * 16; }

// -------------------------------------------------------------- attention

// Scores of every session's keys (k_attn_scores' arithmetic: lane l of a
// 32-lane unit owns channels l, l + 32, ..., summed serially from 0.0, then
// the 32-wide halving tree, times 1/sqrt(HD)), with the group's HPK query
// heads in registers and two keys per unit reduced by one paired tree (each
// total has its operands of the single tree). Block (key blocks, KV head,
// session) takes chunks of 16 consecutive keys (blockIdx.x, + gridDim.x,
// ...): a chunk's key rows are loaded as whole lines (16-byte pieces, each
// row's pieces on consecutive threads) into LDS, the next chunk's loads in
// flight while unit u scores keys 2u and 2u + 1 from there. scores
// [session][q_heads][stride].
template <int HPK, int KJ>
__global__ __launch_bounds__(kBlock) void k_bscores(const uint16_t* __restrict__ q,
                                                    const SessionRows* __restrict__ rows, int64_t key_base, int kvs,
                                                    float scale, float* __restrict__ scores, int stride) {
  constexpr int HD = 32 * KJ, RQ = HD / 8;      // channels, 16-byte pieces per key row
  constexpr int CK = 2 * (kBlock / 32);         // keys per chunk: two per unit
  constexpr int PT = (CK * RQ + kBlock - 1) / kBlock;  // pieces per thread
  __shared__ __align__(16) uint16_t kst[2][CK * HD];
  const int kvh = blockIdx.y, b = blockIdx.z;
  const int q_heads = gridDim.y * HPK;
  const int l32 = threadIdx.x & 31, unit = threadIdx.x >> 5;
  const int64_t keys = (int64_t)rows->position[b] + 1;
  const auto kbase = gmem(rows->cache[b] + key_base + (int64_t)kvh * HD);
  float* sb = scores + (size_t)b * q_heads * stride + (size_t)kvh * HPK * stride;
  float qv[HPK][KJ];
#pragma unroll
  for (int h = 0; h < HPK; ++h)
#pragma unroll
    for (int j = 0; j < KJ; ++j)
      qv[h][j] = bf2f(q[((size_t)b * q_heads + kvh * HPK + h) * HD + l32 + 32 * j]);
  // piece i of this thread: key row (tid + kBlock i) / RQ of the chunk, its
  // 16-byte piece (tid + kBlock i) % RQ
  u32x4 kv[PT];
  auto load = [&](int64_t c0) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int idx = threadIdx.x + kBlock * i;
      if (CK * RQ % kBlock == 0 || idx < CK * RQ) {
        const int64_t key = min<int64_t>(c0 + idx / RQ, keys - 1);
        kv[i] = *reinterpret_cast<const __attribute__((address_space(1))) u32x4*>(kbase + key * kvs +
                                                                                  8 * (idx % RQ));
      }
    }
  };
  auto put = [&](int buf) {
#pragma unroll
    for (int i = 0; i < PT; ++i) {
      const int idx = threadIdx.x + kBlock * i;
      if (CK * RQ % kBlock == 0 || idx < CK * RQ) reinterpret_cast<u32x4*>(kst[buf])[idx] = kv[i];
    }
  };
  const int64_t step = (int64_t)CK * gridDim.x;
  int64_t c0 = (int64_t)CK * blockIdx.x;
  if (c0 >= keys) return;  // uniform per block
  load(c0);
  put(0);
  __syncthreads();
  for (int buf = 0; c0 < keys; c0 += step, buf ^= 1) {
    load(c0 + step);  // unconditional (clamped): a conditional load would drain the queue
    const uint16_t* ka = kst[buf] + (2 * unit) * HD + l32;
    float fa[KJ], fb[KJ];
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      fa[j] = bf2f(ka[32 * j]);
      fb[j] = bf2f(ka[HD + 32 * j]);
    }
    const int64_t kk = c0 + 2 * unit;
#pragma unroll
    for (int h = 0; h < HPK; ++h) {
      float a = 0.0f, c = 0.0f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) {
        a += qv[h][j] * fa[j];
        c += qv[h][j] * fb[j];
      }
      const float v = tree32_pair(a, c);
      if (l32 == 0 && kk < keys) sb[(size_t)h * stride + kk] = v * scale;
      if (l32 == 16 && kk + 1 < keys) sb[(size_t)h * stride + kk + 1] = v * scale;
    }
    put(buf ^ 1);  // the other buffer's readers finished before the last barrier
    __syncthreads();
  }
}

// k_bflash: block (range, head group, session) with one thread per pair of
// channels (c, c + 1: one 4-byte V read per key) and one wave for the
// denominators. kSplit: split sessions only, the group is a KV head's kHPB
// query heads (kHPB = heads per KV head) and the tiles are range r's;
// otherwise sessions at or below their split threshold, the group one query
// head (kHPB = 1) and the tiles all of them (range 0). Tiles run in
// sub-chunks of up to 64: the scores of the sub-chunk staged, each head's
// running maximum per tile (reset at the range start), alpha_t =
// exp(m_{t-1} - m_t), p = exp(s - m_t) (invalid keys p = 0 against key 0's
// value), then per channel and head the chain acc = acc * alpha_t +
// p_0 v_0 + ... + p_7 v_7 and per head den = den * alpha_t + p_0 + ... + p_7
// (k_attn_values' arithmetic), the V values kFlashRing tiles ahead of the
// chains. Split: the range's (m_r, den_r, acc_r[HD]) go to part; single
// chain: the output bf16(bf16(acc / den) * sigmoid(gate)).
constexpr int kFlashSub = 64;  // tiles per sub-chunk
constexpr int kFlashRing = 4;  // tiles of V values in flight per thread

inline int flash_threads(int head_dim) { return (head_dim / 2 + 63) / 64 * 64 + 64; }

template <bool kSplit, int kHPB>
__global__ __launch_bounds__(192) void k_bflash(const float* __restrict__ scores, int stride,
                                                const SessionRows* __restrict__ rows, int64_t value_base, int kvs,
                                                int head_dim, int q_heads, int heads_per_kv,
                                                const uint16_t* __restrict__ qg, float* __restrict__ part,
                                                uint16_t* __restrict__ out) {
  constexpr int HPB = kHPB, D = kFlashRing;
  __shared__ __align__(16) float p[HPB][kFlashSub * 8];
  __shared__ float alpha[HPB][kFlashSub];
  __shared__ float mtile[HPB][kFlashSub];
  __shared__ float mrun[HPB], dfinal[HPB];
  const int b = blockIdx.z, tid = threadIdx.x;
  const int64_t keys = (int64_t)rows->position[b] + 1;
  const int tiles = (int)((keys + 7) >> 3);
  const int64_t sk = rows->split[b];
  const bool split = sk > 0 && keys > sk;
  if (kSplit != split) return;
  const int range_tiles = split ? (tiles + kSplitRanges - 1) / kSplitRanges : tiles;
  const int r = blockIdx.x;
  if (r * range_tiles >= tiles) return;
  const int t_begin = r * range_tiles, t_end = min(tiles, t_begin + range_tiles);
  constexpr int nh = HPB;
  const int h0 = kSplit ? blockIdx.y * heads_per_kv : blockIdx.y;
  const int kvh = h0 / heads_per_kv;
  const int half_pad = (head_dim / 2 + 63) / 64 * 64;
  const bool chan = tid < head_dim / 2;
  const int c = 2 * tid;
  const bool den_lane = tid >= half_pad && tid - half_pad < nh;
  const int dh = tid - half_pad;
  const float ninf = bitsf(0xff800000u);
  const float* sb = scores + (size_t)b * q_heads * stride;
  const auto vb = gmem(reinterpret_cast<const uint32_t*>(rows->cache[b] + value_base + (int64_t)kvh * head_dim +
                                                         (chan ? c : 0)));
  const int kvw = kvs / 2;  // key stride in 4-byte words
  auto vload = [&](int64_t k) { return vb[(k < keys ? k : 0) * kvw]; };
  float acc[HPB][2];
#pragma unroll
  for (int h = 0; h < HPB; ++h) acc[h][0] = acc[h][1] = 0.0f;
  float den = 0.0f;
  if (tid < nh) mrun[tid] = ninf;
  for (int c0 = t_begin; c0 < t_end; c0 += kFlashSub) {
    const int nt = min(kFlashSub, t_end - c0), nk = nt * 8;
    const int64_t k0 = (int64_t)c0 * 8;
    // the first tiles' V values, in flight while the weights are computed
    uint32_t vr[D][8];
    if (chan) {
#pragma unroll
      for (int d = 0; d < D; ++d)
#pragma unroll
        for (int j = 0; j < 8; ++j) vr[d][j] = vload(k0 + 8 * d + j);
    }
    __syncthreads();  // the previous sub-chunk's readers are done
    for (int i = tid; i < nh * nk; i += blockDim.x) {
      const int h = i / nk, kk = i - h * nk;
      const int64_t k = k0 + kk;
      p[h][kk] = k < keys ? sb[(size_t)(h0 + h) * stride + k] : ninf;
    }
    __syncthreads();
    // tile maxima in parallel, then each head's running maximum
    for (int i = tid; i < nh * nt; i += blockDim.x) {
      const int h = i / nt, ti = i - h * nt;
      float tm = ninf;
#pragma unroll
      for (int j = 0; j < 8; ++j) tm = fmaxf(tm, p[h][ti * 8 + j]);
      mtile[h][ti] = tm;
    }
    __syncthreads();
    if (tid < nh) {
      const int h = tid;
      float m = mrun[h];
      for (int i = 0; i < nt; ++i) {
        const float prev = (c0 + i == t_begin) ? ninf : m;
        m = fmaxf(m, mtile[h][i]);
        mtile[h][i] = m;
        alpha[h][i] = prev;  // exponentiated below
      }
      mrun[h] = m;
    }
    __syncthreads();
    for (int i = tid; i < nh * nt; i += blockDim.x) {
      const int h = i / nt, ti = i - h * nt;
      alpha[h][ti] = hexp(alpha[h][ti] - mtile[h][ti]);
    }
    for (int i = tid; i < nh * nk; i += blockDim.x) {
      const int h = i / nk, kk = i - h * nk;
      const int64_t k = k0 + kk;
      p[h][kk] = k < keys ? hexp(p[h][kk] - mtile[h][kk >> 3]) : 0.0f;
    }
    // tiles past nt up to a whole ring group are no-ops: alpha 1 and p 0
    // leave every chain's bits unchanged (x * 1 = x, x + (+-0) = x), so the
    // chain loop below runs whole groups with no runtime guard
    const int ntp = (nt + D - 1) / D * D;
    for (int i = tid; i < nh * (ntp - nt); i += blockDim.x) {
      const int h = i / (ntp - nt), ti = nt + i - h * (ntp - nt);
      alpha[h][ti] = 1.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j) p[h][ti * 8 + j] = 0.0f;
    }
    __syncthreads();
    if (chan) {
      // loads are issued unconditionally (keys past the range are valid
      // rows, keys past the end read key 0): a conditional load would make
      // the next use wait for every load in flight
      for (int i0 = 0; i0 < ntp; i0 += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
          const int i = i0 + d;
          float v0[8], v1[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            v0[j] = lo2f(vr[d][j]);
            v1[j] = hi2f(vr[d][j]);
          }
#pragma unroll
          for (int j = 0; j < 8; ++j) vr[d][j] = vload(k0 + 8 * (i + D) + j);
#pragma unroll
          for (int h = 0; h < HPB; ++h) {
            const f32x4 pa = reinterpret_cast<const f32x4*>(&p[h][i * 8])[0];
            const f32x4 pb = reinterpret_cast<const f32x4*>(&p[h][i * 8])[1];
            const float al = alpha[h][i];
            const float pw[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
            float a0 = acc[h][0] * al, a1 = acc[h][1] * al;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              a0 = a0 + pw[j] * v0[j];
              a1 = a1 + pw[j] * v1[j];
            }
            acc[h][0] = a0;
            acc[h][1] = a1;
          }
        }
      }
    } else if (den_lane) {
      for (int i = 0; i < nt; ++i) {
        den = den * alpha[dh][i];
#pragma unroll
        for (int j = 0; j < 8; ++j) den = den + p[dh][i * 8 + j];
      }
    }
  }
  if (split) {
#pragma unroll
    for (int h = 0; h < nh; ++h) {
      float* pr = part + (((size_t)b * q_heads + h0 + h) * kSplitRanges + r) * (2 + head_dim);
      if (chan) {
        pr[2 + c] = acc[h][0];
        pr[3 + c] = acc[h][1];
      }
      if (den_lane && dh == h) {
        pr[0] = mrun[h];
        pr[1] = den;
      }
    }
  } else {
    if (den_lane) dfinal[dh] = den;
    __syncthreads();
    if (chan) {
#pragma unroll
      for (int h = 0; h < nh; ++h) {
        const int head = h0 + h;
        const uint16_t* gr = qg + (size_t)b * 2 * q_heads * head_dim + (size_t)head * 2 * head_dim + head_dim + c;
        uint16_t* o = out + (size_t)b * q_heads * head_dim + head * head_dim + c;
        o[0] = f2bf(rbf(acc[h][0] / dfinal[h]) * sigmoid(bf2f(gr[0])));
        o[1] = f2bf(rbf(acc[h][1] / dfinal[h]) * sigmoid(bf2f(gr[1])));
      }
    }
  }
}

// Merge of a split session's ranges per (query head, session), one thread
// per channel: M = max_r m_r, w_r = exp(m_r - M) (computed once per range),
// then in ascending range order den = 0 + den_r w_r, acc = 0 + acc_r w_r;
// out = bf16(bf16(acc / den) * sigmoid(gate)).
__global__ __launch_bounds__(256) void k_bmerge(const float* __restrict__ part, const SessionRows* __restrict__ rows,
                                                int head_dim, int q_heads, const uint16_t* __restrict__ qg,
                                                uint16_t* __restrict__ out) {
  __shared__ float wr[kSplitRanges], mr[kSplitRanges], dr[kSplitRanges];
  __shared__ float top_s, den_s;
  const int head = blockIdx.x, b = blockIdx.y, c = threadIdx.x;
  const int64_t keys = (int64_t)rows->position[b] + 1;
  const int64_t sk = rows->split[b];
  if (!(sk > 0 && keys > sk)) return;  // block-uniform
  const int tiles = (int)((keys + 7) >> 3);
  const int range_tiles = (tiles + kSplitRanges - 1) / kSplitRanges;
  const int nranges = (tiles + range_tiles - 1) / range_tiles;
  const float* pr = part + ((size_t)b * q_heads + head) * kSplitRanges * (2 + head_dim);
  if (c < nranges) {
    mr[c] = pr[(size_t)c * (2 + head_dim)];
    dr[c] = pr[(size_t)c * (2 + head_dim) + 1];
  }
  __syncthreads();
  if (c == 0) {
    float top = bitsf(0xff800000u);
    for (int r = 0; r < nranges; ++r) top = fmaxf(top, mr[r]);
    top_s = top;
  }
  __syncthreads();
  if (c < nranges) wr[c] = hexp(mr[c] - top_s);
  __syncthreads();
  if (c == 0) {
    float den = 0.0f;
    for (int r = 0; r < nranges; ++r) den = den + dr[r] * wr[r];
    den_s = den;
  }
  float acc = 0.0f;
  if (c < head_dim) {
    constexpr int G = 16;
    for (int r0 = 0; r0 < nranges; r0 += G) {
      float a[G];
#pragma unroll
      for (int g = 0; g < G; ++g) a[g] = pr[(size_t)min(r0 + g, nranges - 1) * (2 + head_dim) + 2 + c];
#pragma unroll
      for (int g = 0; g < G; ++g)
        if (r0 + g < nranges) acc = acc + a[g] * wr[r0 + g];
    }
  }
  __syncthreads();
  if (c < head_dim) {
    const float gate = sigmoid(bf2f(qg[(size_t)b * 2 * q_heads * head_dim + (size_t)head * 2 * head_dim + head_dim + c]));
    out[(size_t)b * q_heads * head_dim + head * head_dim + c] = f2bf(rbf(acc / den_s) * gate);
  }
}

}  // namespace cq35
