// Persistent decode step for the MoE hybrid: one launch per token.
//
// The per-token work of the reference (src/qwen/qwen35.rs:1395-1465: embedding,
// 40 layers, head) is a chain of about 250 dependent phases, each of which
// streams a weight slice that does not depend on the chain. A kernel per
// phase pays its launch and its first-load latency on the critical path.
// Here one grid of one block per CU runs every phase, and each block issues
// the weight loads of its next phase *before* it waits for that phase's
// inputs, so weight streaming overlaps the exchange latency.
//
// Exchange. Every activation that crosses blocks is written as 64-bit words
// (32-bit payload | 32-bit step tag) with device-coherent stores; consumers
// poll the words themselves until every tag equals the step's tag. There are
// no flags and no fences: a word is valid exactly when its tag matches.
// Each (layer, activation) has its own buffer, written once per step, so no
// address is read before it is written within a launch. BF16 activations
// travel two per word (element 2i in the low half), F32 ones one per word.
//
// Every wait is bounded: a thread that polls longer than the spin limit
// raises the block's abort flag and the global error word, after which every
// wait of every block returns at once, so the grid always drains.
//
// Arithmetic and reduction orders are those of the per-kernel path
// (gemv.h, layers.h, attention.h), bit for bit.
#pragma once

#include "attention.h"
#include "layers.h"

namespace cq35 {

constexpr int kMT = 512;       // threads per block
constexpr int kMW = kMT / 64;  // waves per block

// Static per-wave work maxima (checked on the host for every shape).
constexpr int kPairsA = 4;     // projection row pairs per wave
constexpr int kPairsG = 2;     // gate/up row pairs per wave
constexpr int kDownJ = 64;     // routed dwords per lane in the down projection
constexpr int kDownSJ = 16;    // shared dwords per lane
constexpr int kOutJ = 32;      // dwords per lane per row of the output projections
constexpr int kRouterJ = 32;   // router floats per lane
constexpr int kChunkKeys = 512;  // attention keys staged per chunk

struct MegaLayer {
  int full;
  const float* in_norm;
  const uint16_t* seg_w[4];
  int seg_rows[4];
  // linear (Gated DeltaNet)
  const float* dt;
  const float* a;
  const float* gnorm;
  const float* conv_w;
  int64_t conv_base;   // cache element offset of the conv history
  int64_t state_base;  // cache element offset of the recurrent state
  // full attention
  const float* qnorm;
  const float* knorm;
  int64_t key_base, value_base;
  // both
  const uint16_t* out_w;  // ssm_out / attn_output, [H, cols]
  const float* post_norm;
  const float* router;
  const float* shared_gate;
  const uint16_t *gate_exps, *up_exps, *down_exps, *sgate, *sup, *sdown;
  // tagged activation words of this layer
  uint64_t* x_h;       // input hidden row (H/2); unused for layer 0
  uint64_t* x_proj;    // projection outputs (rows/2)
  uint64_t* x_mix;     // gated core (VS/2) or gated attention context (QS/2)
  uint64_t* x_attn;    // residual after the mixer (H/2)
  uint64_t* x_router;  // E+1 F32 logits
  uint64_t* x_active;  // (K*I+SI)/2
  uint64_t* x_scores;  // Q * capacity F32 scores (full layers)
  uint64_t* x_out;     // output hidden row (H/2) = next layer's x_h
};

struct MegaArgs {
  const MegaLayer* layers;
  int L;
  int H, V, Q, KVH, HD, R, KH, KD, VH, VD, KS, VS, QKV, QS, KVS, E, K, I, SI;
  float eps, attn_scale, delta_scale;
  int64_t cap;
  const uint16_t* embed;
  const float* out_norm;
  const uint16_t* head;
  const float* freq;
  uint16_t* cache;
  const uint64_t* params;  // [start, token, step tag]
  const uint64_t* x_final; // hidden row after the last layer (H/2 words)
  uint16_t* logits;
  unsigned long long* best;
  unsigned* error;
  unsigned spin_limit;
};

// LDS carve-up (bytes); the "big" area is reused by the phases that need it.
constexpr int kLdsXn = 0;          // normalised input row, BF16 quads (H <= 2048)
constexpr int kLdsXr = 4096;       // raw hidden row (layer input; mixer residual)
constexpr int kLdsXa = 8192;       // raw post-mixer row (router input; FFN residual)
constexpr int kLdsVec = 12288;     // polled words (4096)
constexpr int kLdsMisc = 28672;    // logits, ids, probs, reductions
constexpr int kLdsBig = 36864;
constexpr int kLdsBigBytes = 53248;
constexpr int kMegaLds = kLdsBig + kLdsBigBytes;

struct MegaMisc {
  float logits[1025];
  int ids[64];
  float probs[64];
  float chosen[64];
  float red[8];
  float scalars[8];
  int abort;
  int any_nan;
};
static_assert(sizeof(MegaMisc) <= kLdsBig - kLdsMisc, "misc LDS");

extern __shared__ __align__(16) unsigned char mega_lds[];

// Pointers read from the argument tables are generic; every HBM access goes
// through the global address space so it compiles to global (not flat)
// memory instructions.
#define CQ35_GLOBAL __attribute__((address_space(1)))
#define CQ35_CONST __attribute__((address_space(4)))
#define CQ35_LDS __attribute__((address_space(3)))
template <typename T>
__device__ __forceinline__ CQ35_GLOBAL T* G(T* p) {
  return (CQ35_GLOBAL T*)p;
}
template <typename T>
__device__ __forceinline__ const CQ35_GLOBAL T* G(const T* p) {
  return (const CQ35_GLOBAL T*)p;
}


// Per-thread view of one phase: the arguments (device memory, read through
// the scalar cache), the step tag, thread coordinates and the LDS carve-up.
// Phases are separate functions that rebuild it, so nothing of it lives in
// private memory across calls.
struct Mega {
  const CQ35_CONST MegaArgs& a;
  uint32_t tag;
  int tid, lane, wave, gw, nw;
  u32x4* xn;
  uint16_t* xr;
  uint16_t* xa;
  uint32_t* vec;
  MegaMisc* misc;
  unsigned char* big;
};

// An opaque copy of a uniform pointer, kept in scalar registers: loads
// through it cannot be hoisted out of the phase that makes the copy, which
// keeps every phase's scalar state local to the phase.
// The tables are written by the host before the launch and never by the
// kernel, so they are read through the constant address space (scalar loads).
template <typename T>
__device__ __forceinline__ const CQ35_CONST T* phase_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  asm volatile("" : "+s"(lo), "+s"(hi));
  return (const CQ35_CONST T*)(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ Mega make_mega(const MegaArgs* pa, uint32_t tag) {
  const CQ35_CONST MegaArgs* a = phase_ptr(pa);
  // per-lane arithmetic is recomputed in every phase instead of being hoisted
  // out of the layer loop and held in registers across all phases
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  // wave-level indices are uniform: keep them in scalar registers so weight
  // rows get scalar base addresses (one 32-bit lane offset per load)
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gw = __builtin_amdgcn_readfirstlane((int)blockIdx.x * kMW + wave);
  const int nw = __builtin_amdgcn_readfirstlane((int)gridDim.x * kMW);
  return Mega{*a,
              tag,
              tid,
              tid & 63,
              wave,
              gw,
              nw,
              reinterpret_cast<u32x4*>(mega_lds + kLdsXn),
              reinterpret_cast<uint16_t*>(mega_lds + kLdsXr),
              reinterpret_cast<uint16_t*>(mega_lds + kLdsXa),
              reinterpret_cast<uint32_t*>(mega_lds + kLdsVec),
              reinterpret_cast<MegaMisc*>(mega_lds + kLdsMisc),
              mega_lds + kLdsBig};
}

// ------------------------------------------------------------ exchange words

__device__ __forceinline__ uint64_t word_load(const uint64_t* p) {
  return __hip_atomic_load(G(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void word_store(uint64_t* p, uint32_t payload, uint32_t tag) {
  __hip_atomic_store(G(p), ((uint64_t)tag << 32) | payload, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ bool word_ready(uint64_t w, uint32_t tag) {
  return (uint32_t)(w >> 32) == tag;
}

__device__ __forceinline__ volatile CQ35_LDS int* abort_flag(const Mega& m) {
  return (volatile CQ35_LDS int*)&m.misc->abort;
}
__device__ __forceinline__ bool mega_aborted(const Mega& m) { return *abort_flag(m) != 0; }

// Spin bookkeeping of one polling loop: true when the wait must stop.
__device__ __forceinline__ bool spin_exhausted(const Mega& m, unsigned& spins) {
  if (mega_aborted(m)) return true;
  ++spins;
  if ((spins & 255u) == 0 &&
      __hip_atomic_load(G(m.a.error), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0) {
    *abort_flag(m) = 1;
    return true;
  }
  if (spins > m.a.spin_limit) {
    __hip_atomic_fetch_or(G(m.a.error), 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *abort_flag(m) = 1;
    return true;
  }
  return false;
}

// Poll n words (word i = src_index(i)) until every tag matches, then write
// the payloads to dst[i]. Up to MAXW words per thread; block-wide; ends with
// a barrier.
template <int MAXW, typename Index>
__device__ __forceinline__ void poll_words(const Mega& m, const uint64_t* src, int n, Index src_index,
                                           uint32_t* dst) {
  uint64_t v[MAXW];
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = m.tid + kMT * j;
    v[j] = i < n ? word_load(src + src_index(i)) : ((uint64_t)m.tag << 32);
  }
  unsigned spins = 0;
  while (true) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) ready &= word_ready(v[j], m.tag);
    if (ready || spin_exhausted(m, spins)) break;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) {
      const int i = m.tid + kMT * j;
      if (!word_ready(v[j], m.tag)) v[j] = word_load(src + src_index(i));
    }
  }
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = m.tid + kMT * j;
    if (i < n) dst[i] = (uint32_t)v[j];
  }
  __syncthreads();
}

struct Identity {
  __device__ __forceinline__ int operator()(int i) const { return i; }
};

// Poll one word per calling thread (any subset of threads); returns the payload.
__device__ __forceinline__ uint32_t poll_one(const Mega& m, const uint64_t* p) {
  uint64_t v = word_load(p);
  unsigned spins = 0;
  while (!word_ready(v, m.tag) && !spin_exhausted(m, spins)) v = word_load(p);
  return (uint32_t)v;
}

// ------------------------------------------------------- normalised input

// qwen35.normalize (qwen35.hex:912-977) of the raw row in `raw` (H <= 2048)
// into m.xn, with the norm weights prefetched by thread t < 256 for octet t.
// The adjacent-pair tree over the padded width equals the octet tree, the
// 64-lane shuffle tree and ((w0 + w1) + (w2 + w3)) over waves 0-3 (threads
// past H/8 hold +0, and joining a zero subtree is exact).
__device__ __forceinline__ void norm_row(const Mega& m, const uint16_t* raw, f32x4 w0, f32x4 w1) {
  const int H = m.a.H;
  const bool own = m.tid < (H >> 3);
  u32x4 x = {0u, 0u, 0u, 0u};
  if (own) x = reinterpret_cast<const u32x4*>(raw)[m.tid];
  float t = own ? octet_squares(x) : 0.0f;
  t = t + lane_down<1>(t);
  t = t + lane_down<2>(t);
  t = t + lane_down<4>(t);
  t = t + lane_down<8>(t);
  t = t + lane_down<16>(t);
  t = t + lane_down<32>(t);
  if (m.lane == 0 && m.wave < 4) m.misc->red[m.wave] = t;
  __syncthreads();
  const float sum = (m.misc->red[0] + m.misc->red[1]) + (m.misc->red[2] + m.misc->red[3]);
  const float inverse = 1.0f / nsqrt(sum / (float)H + m.a.eps);
  if (own) m.xn[m.tid] = octet_scale(x, inverse, w0, w1);
  __syncthreads();
}

__device__ __forceinline__ void norm_weights(const Mega& m, const float* w, f32x4& w0, f32x4& w1) {
  const int o = min(m.tid, (m.a.H >> 3) - 1);
  w0 = G(reinterpret_cast<const f32x4*>(w))[2 * o];
  w1 = G(reinterpret_cast<const f32x4*>(w))[2 * o + 1];
}

// Raw hidden row of layer l into `raw`: the embedding row for layer 0,
// otherwise the previous layer's output words.
__device__ __forceinline__ void load_hidden(const Mega& m, const uint64_t* words, uint16_t* raw,
                                            bool embedding) {
  const int H = m.a.H;
  if (embedding) {
    const uint64_t token = G(m.a.params)[1];
    const u32x4* row = reinterpret_cast<const u32x4*>(m.a.embed + token * (uint64_t)H);
    if (m.tid < (H >> 3)) reinterpret_cast<u32x4*>(raw)[m.tid] = G(row)[m.tid];
    __syncthreads();
  } else {
    poll_words<2>(m, words, H >> 1, Identity{}, reinterpret_cast<uint32_t*>(raw));
  }
}

// --------------------------------------------------- split-pair primitives

// Loads at a wave-uniform base plus a 32-bit per-lane byte offset (scalar
// base address, one VGPR of address per load).
__device__ __forceinline__ u32x4 ldq_at(const void* base, uint32_t byte_off) {
  return *G(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(base) + byte_off));
}
__device__ __forceinline__ uint32_t ldd_at(const void* base, uint32_t byte_off) {
  return *G(reinterpret_cast<const uint32_t*>(reinterpret_cast<const char*>(base) + byte_off));
}
__device__ __forceinline__ float ldf_at(const void* base, uint32_t byte_off) {
  return *G(reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + byte_off));
}

__device__ __forceinline__ void pair_acc(float& lo, float& hi, uint32_t x, uint32_t w) {
  lo += lo2f(x) * lo2f(w);
  hi += hi2f(x) * hi2f(w);
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

// -------------------------------------------------- phase: S256 projection

__device__ __forceinline__ const uint16_t* seg_row(const CQ35_CONST MegaLayer& Ly, int row, int cols) {
  const int e0 = Ly.seg_rows[0], e1 = e0 + Ly.seg_rows[1], e2 = e1 + Ly.seg_rows[2];
  const int s = row < e0 ? 0 : row < e1 ? 1 : row < e2 ? 2 : 3;
  const int local = row - (s == 0 ? 0 : s == 1 ? e0 : s == 2 ? e1 : e2);
  const uint16_t* w = s == 0 ? Ly.seg_w[0] : s == 1 ? Ly.seg_w[1] : s == 2 ? Ly.seg_w[2] : Ly.seg_w[3];
  return w + (size_t)local * cols;
}

// Normalised hidden row x grouped BF16 matrices (group-project,
// group_projection.hex:3-97): S256 split pairs, a physical lane holding
// reference lanes 4q..4q+3; row pairs (2p, 2p+1) per output word.
__device__ __forceinline__ void phase_project(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int l) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const int H = m.a.H, quads = H >> 3;
  const int total = Ly.seg_rows[0] + Ly.seg_rows[1] + Ly.seg_rows[2] + Ly.seg_rows[3];
  const int pairs = total >> 1;
  u32x4 wv[kPairsA][2][4];
#pragma unroll
  for (int k = 0; k < kPairsA; ++k) {
    const int p = m.gw + m.nw * k;
    if (p < pairs) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint16_t* w = seg_row(Ly, 2 * p + r, H);
#pragma unroll
        for (int j = 0; j < 4; ++j) wv[k][r][j] = ldq_at(w, (uint32_t)min(m.lane + 64 * j, quads - 1) * 16u);
      }
    }
  }
  f32x4 w0, w1;
  norm_weights(m, Ly.in_norm, w0, w1);
  load_hidden(m, Ly.x_h, m.xr, l == 0);
  norm_row(m, m.xr, w0, w1);
#pragma unroll
  for (int k = 0; k < kPairsA; ++k) {
    const int p = m.gw + m.nw * k;
    if (p < pairs) {
      float v[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        Quad acc;
        quad_zero(acc);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (m.lane + 64 * j < quads) quad_acc(acc, m.xn[m.lane + 64 * j], wv[k][r][j]);
        v[r] = quad_tree<64>(acc);
      }
      if (m.lane == 0) word_store(Ly.x_proj + p, pack_bf(f2bf(v[0]), f2bf(v[1])), m.tag);
    }
  }
}

// ------------------------------------------- phase: Gated DeltaNet (linear)

// One block per value head h (key head h % KH): the 4-tap convolution of the
// head's q, k and v channels (linear_prepare.hex:2-64), serial L2 norms of q
// and k (linear_prepare.hex:84-131), the gates (fused_delta.hex:1-20), the
// delta step of the head's VD channels with the state staged in LDS
// (cached_delta.hex:69-168, D32 trees) and the gated RMSNorm x SiLU(z)
// (cooperative_norm.hex:139-182). The v channels' conv history is written
// here; the q and k channels' history is shared with the other value heads
// of the key head and is written by block kh in the next phase, after every
// reader has finished.
struct DeltaLds {
  float conv[512];      // conv outputs, channel order q | k | v (as floats of BF16)
  float sq[256];        // squares for the serial sums
  uint16_t qhat[128];
  uint16_t khat[128];
  uint16_t core[128];
  uint16_t raw_qk[256]; // raw q | k of the key head (history written next phase)
  float gates[4];       // decay, rate
};
constexpr int kDeltaState = 8192;  // offset of the state rows in the big area
static_assert(sizeof(DeltaLds) <= kDeltaState, "delta LDS");

__device__ __forceinline__ void phase_delta(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int h = blockIdx.x;
  if (h >= a.VH) return;  // uniform per block
  const int KD = a.KD, VD = a.VD, kh = h % a.KH;
  const int nch = 2 * KD + VD;
  DeltaLds* d = reinterpret_cast<DeltaLds*>(m.big);
  uint16_t* state = reinterpret_cast<uint16_t*>(m.big + kDeltaState);
  uint16_t* st_g = a.cache + Ly.state_base + (size_t)h * VD * KD;
  // prefetch: state rows, conv taps, history, gate parameters
  const int squads = (VD * KD) >> 3;
  u32x4 sv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j)
    sv[j] = ldq_at(st_g, (uint32_t)min(m.tid + kMT * j, squads - 1) * 16u);
  const int64_t position = (int64_t)G(a.params)[0];
  int ch = 0;
  if (m.tid < KD) ch = kh * KD + m.tid;
  else if (m.tid < 2 * KD) ch = a.KS + kh * KD + (m.tid - KD);
  else ch = 2 * a.KS + h * VD + (m.tid - 2 * KD);
  const bool conv_thread = m.tid < nch;
  f32x4 taps_w = {0.f, 0.f, 0.f, 0.f};
  float hist[3] = {0.f, 0.f, 0.f};
  const uint16_t* history = a.cache + Ly.conv_base;
  if (conv_thread) {
    taps_w = G(reinterpret_cast<const f32x4*>(Ly.conv_w))[ch];
#pragma unroll
    for (int k = 0; k < 3; ++k) hist[k] = bf2f(G(history)[((position + k) % 3) * a.QKV + ch]);
  }
  const float dt = G(Ly.dt)[h], aa = G(Ly.a)[h];
  const float gw = m.tid < VD ? G(Ly.gnorm)[m.tid] : 0.0f;
  // inputs: q | k | v of this head, z, alpha, beta (projection words)
  const int qw = KD >> 1, vw = VD >> 1;
  const int zbase = a.QKV, abase = a.QKV + a.VS, bbase = abase + a.VH;
  const int nwords = 2 * qw + 2 * vw + 2;
  auto index = [&](int i) -> int {
    if (i < qw) return ((kh * KD) >> 1) + i;
    if (i < 2 * qw) return ((a.KS + kh * KD) >> 1) + (i - qw);
    if (i < 2 * qw + vw) return ((2 * a.KS + h * VD) >> 1) + (i - 2 * qw);
    if (i < 2 * qw + 2 * vw) return ((zbase + h * VD) >> 1) + (i - 2 * qw - vw);
    if (i == 2 * qw + 2 * vw) return (abase + h) >> 1;
    return (bbase + h) >> 1;
  };
  poll_words<1>(m, Ly.x_proj, nwords, index, m.vec);
  const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (m.tid + kMT * j < squads) reinterpret_cast<u32x4*>(state)[m.tid + kMT * j] = sv[j];
  // convolution (linear_prepare.hex:2-64)
  if (conv_thread) {
    const uint16_t current = in16[m.tid];
    float taps[3];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
      const int64_t p = position + k;
      const float w = k == 0 ? taps_w.x : k == 1 ? taps_w.y : taps_w.z;
      taps[k] = (p < 3 ? 0.0f : hist[k]) * w;
    }
    const float tap3 = bf2f(current) * taps_w.w;
    const float sum = (taps[0] + taps[2]) + (taps[1] + tap3);
    const float out = bf2f(f2bf(silu(rbf(sum))));
    d->conv[m.tid] = out;
    if (m.tid < 2 * KD) {
      d->sq[m.tid] = out * out;
      d->raw_qk[m.tid] = current;
    } else {
      // v history: read by this block only
      G(a.cache)[Ly.conv_base + (position % 3) * a.QKV + ch] = current;
    }
  }
  __syncthreads();
  // serial L2 sums (q: thread 0, k: thread 64) and the gates (thread 128)
  if (m.tid == 0 || m.tid == 64) {
    const float* s = d->sq + (m.tid == 0 ? 0 : KD);
    float total = 0.0f;
    for (int i = 0; i < KD; ++i) total += s[i];
    d->gates[2 + (m.tid == 0 ? 0 : 1)] = nsqrt(total + bitsf(0x358637bdu));
  } else if (m.tid == 128) {
    const uint16_t alpha = in16[2 * (2 * qw + 2 * vw) + ((abase + h) & 1)];
    const uint16_t beta = in16[2 * (2 * qw + 2 * vw + 1) + ((bbase + h) & 1)];
    const float time_step = softplus(bf2f(alpha) + dt);
    d->gates[0] = hexp(rbf(time_step * aa));
    d->gates[1] = rbf(sigmoid(bf2f(beta)));
  }
  __syncthreads();
  if (m.tid < 2 * KD) {
    const float norm = d->gates[2 + (m.tid < KD ? 0 : 1)];
    const uint16_t r = f2bf(d->conv[m.tid] / norm);
    if (m.tid < KD) d->qhat[m.tid] = r;
    else d->khat[m.tid - KD] = r;
  }
  __syncthreads();
  // delta step: 16 channels per pass, 32 lanes per channel
  const float decay = d->gates[0], rate = d->gates[1];
  const int sub = m.tid >> 5, l32 = m.tid & 31, kj = KD >> 5;
  for (int c0 = 0; c0 < VD; c0 += kMT / 32) {
    const int c = c0 + sub;
    const bool valid = c < VD;
    const int cc = valid ? c : 0;
    float old[4], kv[4];
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < kj) {
        const int i = l32 + 32 * j;
        old[j] = bf2f(state[cc * KD + i]);
        kv[j] = bf2f(d->khat[i]);
        acc += old[j] * kv[j];
      }
    }
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) acc += __shfl_down(acc, s, 32);
    const float total = __shfl(acc, 0, 32);
    const float value = d->conv[2 * KD + cc];
    const float delta = (value - total * decay) * rate;
    float acc2 = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < kj) {
        const int i = l32 + 32 * j;
        const float next = old[j] * decay + kv[j] * delta;
        if (valid) state[cc * KD + i] = f2bf(next);
        acc2 += next * bf2f(d->qhat[i]);
      }
    }
#pragma unroll
    for (int s = 16; s >= 1; s >>= 1) acc2 += __shfl_down(acc2, s, 32);
    if (l32 == 0 && valid) d->core[c] = f2bf(acc2 * a.delta_scale);
  }
  __syncthreads();
  // state write-back (this block's head only; read again next step)
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (m.tid + kMT * j < squads)
      G(reinterpret_cast<u32x4*>(st_g))[m.tid + kMT * j] = reinterpret_cast<const u32x4*>(state)[m.tid + kMT * j];
  // gated RMSNorm with a serial sum (cooperative_norm.hex:139-182)
  if (m.tid < VD) {
    const float v = bf2f(d->core[m.tid]);
    d->sq[m.tid] = v * v;
  }
  __syncthreads();
  if (m.tid == 0) {
    float total = 0.0f;
    for (int i = 0; i < VD; ++i) total += d->sq[i];
    d->gates[2] = total;
  }
  __syncthreads();
  if (m.tid < VD) {
    const float rms = nsqrt(d->gates[2] / (float)VD + a.eps);
    const float normalized = bf2f(d->core[m.tid]) / rms;
    const uint16_t zb = in16[2 * KD + VD + m.tid];
    const float gate = silu(bf2f(zb));
    const uint16_t y = f2bf((normalized * gw) * gate);
    const uint16_t other = (uint16_t)__shfl_down((int)y, 1, 64);
    if ((m.tid & 1) == 0) word_store(Ly.x_mix + ((h * VD + m.tid) >> 1), pack_bf(y, other), m.tag);
  }
}

// -------------------------------- phase: output projection + residual (S64)

// bf16(bf16(tree64(x . w_r)) (+) residual_r) (qwen3.fused.residual,
// simt.hex:442-538) over the polled mixer output `x_mix` (cols BF16), one
// reference lane per physical lane, two rows per wave. Blocks kh < KH of a
// linear layer also write the q and k conv history of key head kh.
__device__ __forceinline__ void phase_outproj(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int cols) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int H = a.H, np = cols >> 1, nj = (np + 63) >> 6;
  const int prow = m.gw;  // row pair
  uint32_t wv[2][kOutJ];
  if (prow < (H >> 1)) {
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint16_t* w = Ly.out_w + (size_t)(2 * prow + r) * cols;
#pragma unroll
      for (int j = 0; j < kOutJ; ++j)
        if (j < nj) wv[r][j] = ldd_at(w, (uint32_t)min(m.lane + 64 * j, np - 1) * 4u);
    }
  }
  poll_words<4>(m, Ly.x_mix, np, Identity{}, m.vec);
  if (!Ly.full && (int)blockIdx.x < a.KH && blockIdx.x < (unsigned)a.VH) {
    // q and k history of key head kh = blockIdx.x (its raw values are still in
    // this block's LDS from the previous phase).
    const DeltaLds* d = reinterpret_cast<const DeltaLds*>(m.big);
    const int kh = blockIdx.x, KD = a.KD;
    const int64_t slot = ((int64_t)G(a.params)[0] % 3) * a.QKV;
    if (m.tid < 2 * KD) {
      const int ch = m.tid < KD ? kh * KD + m.tid : a.KS + kh * KD + (m.tid - KD);
      G(a.cache)[Ly.conv_base + slot + ch] = d->raw_qk[m.tid];
    }
  }
  if (prow < (H >> 1)) {
    float v[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      float lo = 0.0f, hi = 0.0f;
#pragma unroll
      for (int j = 0; j < kOutJ; ++j) {
        const int p = m.lane + 64 * j;
        if (j < nj && p < np) pair_acc(lo, hi, m.vec[p], wv[r][j]);
      }
      v[r] = tree64_lanes(lo + hi);
    }
    if (m.lane == 0) {
      const uint16_t o0 = bf_add(f2bf(v[0]), m.xr[2 * prow]);
      const uint16_t o1 = bf_add(f2bf(v[1]), m.xr[2 * prow + 1]);
      word_store(Ly.x_attn + prow, pack_bf(o0, o1), m.tag);
    }
  }
  __syncthreads();
}

// ----------------------------------------------- phase: MoE router (S32 F32)

// Every block normalises the post-mixer row (post_attention_norm) into m.xn
// for the router and the gate/up phase and keeps the raw row for the FFN
// residual. Waves gw <= E compute router row gw (moe.hex:4-84): physical lane
// 2r + h runs reference lane r's low (h = 0) or high (h = 1) accumulator over
// floats 64k + lane.
__device__ __forceinline__ void phase_router(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int H = a.H, rows = a.E + 1, nj = (H + 63) >> 6;
  float wv[kRouterJ];
  const bool has_row = m.gw < rows;
  if (has_row) {
    const float* w = m.gw < a.E ? Ly.router + (size_t)m.gw * H : Ly.shared_gate;
#pragma unroll
    for (int j = 0; j < kRouterJ; ++j)
      if (j < nj) wv[j] = ldf_at(w, (uint32_t)min(64 * j + m.lane, H - 1) * 4u);
  }
  f32x4 w0, w1;
  norm_weights(m, Ly.post_norm, w0, w1);
  poll_words<2>(m, Ly.x_attn, H >> 1, Identity{}, reinterpret_cast<uint32_t*>(m.xa));
  norm_row(m, m.xa, w0, w1);
  if (has_row) {
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(m.xn);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouterJ; ++j) {
      const int i = 64 * j + m.lane;
      if (j < nj && i < H) acc += bf2f(xe[i]) * wv[j];
    }
    float v = acc + lane_down<1>(acc);
    v += lane_down<32>(v);
    v += lane_down<16>(v);
    v += lane_down<8>(v);
    v += lane_down<4>(v);
    v += lane_down<2>(v);
    if (m.lane == 0) word_store(Ly.x_router + m.gw, fbits(v), m.tag);
  }
}

// ----------------------------------------- phase: top-k select + gate / up

// Every block ranks the experts itself (moe.hex:86-252): without NaNs, top-k
// rounds of a wave-wide (value, lowest index) maximum; otherwise the
// reference's rank formula. Then dual S256 gate/up rows over the selected
// and shared experts (moe.hex:254-333): routed bf16(silu(g) * u * p_slot),
// shared bf16(bf16(bf16(silu(g)) * u) * sigmoid(shared logit)).
__device__ __forceinline__ void select_experts(const Mega& m) {
  const CQ35_CONST MegaArgs& a = m.a;
  MegaMisc* s = m.misc;
  const int E = a.E, K = a.K;
  if (m.tid == 0) s->any_nan = 0;
  __syncthreads();
  for (int e = m.tid; e < E; e += kMT)
    if (s->logits[e] != s->logits[e]) s->any_nan = 1;
  __syncthreads();
  if (!s->any_nan) {
    if (m.wave == 0) {
      unsigned long long taken = 0;  // bit j: lane's j-th candidate chosen (E <= 4096)
      for (int k = 0; k < K; ++k) {
        unsigned long long mine = 0ull;
        for (int j = 0, e = m.lane; e < E; ++j, e += 64) {
          if ((taken >> j) & 1ull) continue;
          const float le = s->logits[e];
          const uint32_t u = le == 0.0f ? 0u : fbits(le);
          const uint32_t ordered = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
          const unsigned long long key =
              ((unsigned long long)ordered << 32) | (0xffffffffu - (uint32_t)e);
          mine = key > mine ? key : mine;
        }
        unsigned long long best = mine;
#pragma unroll
        for (int sh = 32; sh >= 1; sh >>= 1) {
          const unsigned long long o = __shfl_xor(best, sh, 64);
          best = o > best ? o : best;
        }
        const int e = (int)(0xffffffffu - (uint32_t)(best & 0xffffffffu));
        if ((e & 63) == m.lane) taken |= 1ull << (e >> 6);
        if (m.lane == 0) {
          s->ids[k] = e;
          s->chosen[k] = s->logits[e];
        }
      }
    }
  } else {
    for (int e = m.tid; e < E; e += kMT) {
      const float le = s->logits[e];
      int rank = 0;
      for (int i = 0; i < E; ++i) {
        const float o = s->logits[i];
        rank += (o > le) ? 1 : ((i < e && !(le > o)) ? 1 : 0);
      }
      if (rank < K) {
        s->ids[rank] = e;
        s->chosen[rank] = le;
      }
    }
  }
  __syncthreads();
  if (m.wave == 0) {
    const float ex = m.lane < K ? hexp(s->chosen[m.lane] - s->chosen[0]) : 0.0f;
    float den = 0.0f;
    for (int j = 0; j < K; ++j) den = den + __shfl(ex, j, 64);
    if (m.lane < K) s->probs[m.lane] = ex / den;
    if (m.lane == 0) s->scalars[0] = sigmoid(s->logits[E]);
  }
  __syncthreads();
}

__device__ __forceinline__ void gate_rows(const Mega& m, const CQ35_CONST MegaLayer& Ly, int row,
                                          const uint16_t*& g, const uint16_t*& u) {
  const CQ35_CONST MegaArgs& a = m.a;
  const int routed = a.K * a.I;
  if (row < routed) {
    const int slot = row / a.I;
    const int id = __builtin_amdgcn_readfirstlane(m.misc->ids[slot]);
    const size_t e = (size_t)id * a.I + (row - slot * a.I);
    g = Ly.gate_exps + e * a.H;
    u = Ly.up_exps + e * a.H;
  } else {
    g = Ly.sgate + (size_t)(row - routed) * a.H;
    u = Ly.sup + (size_t)(row - routed) * a.H;
  }
}

__device__ __forceinline__ void phase_gate_up(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int H = a.H, quads = H >> 3;
  const int routed = a.K * a.I, pairs = (routed + a.SI) >> 1;
  u32x4 gv[kPairsG][2][4], uv[kPairsG][2][4];
  // the shared expert's rows do not depend on the routing: load them first
#pragma unroll
  for (int k = 0; k < kPairsG; ++k) {
    const int p = m.gw + m.nw * k;
    if (p < pairs && 2 * p >= routed) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint16_t* g = Ly.sgate + (size_t)(2 * p + r - routed) * H;
        const uint16_t* u = Ly.sup + (size_t)(2 * p + r - routed) * H;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t off = (uint32_t)min(m.lane + 64 * j, quads - 1) * 16u;
          gv[k][r][j] = ldq_at(g, off);
          uv[k][r][j] = ldq_at(u, off);
        }
      }
    }
  }
  poll_words<3>(m, Ly.x_router, a.E + 1, Identity{}, reinterpret_cast<uint32_t*>(m.misc->logits));
  select_experts(m);
#pragma unroll
  for (int k = 0; k < kPairsG; ++k) {
    const int p = m.gw + m.nw * k;
    if (p < pairs && 2 * p < routed) {
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        const uint16_t *g, *u;
        gate_rows(m, Ly, 2 * p + r, g, u);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const uint32_t off = (uint32_t)min(m.lane + 64 * j, quads - 1) * 16u;
          gv[k][r][j] = ldq_at(g, off);
          uv[k][r][j] = ldq_at(u, off);
        }
      }
    }
  }
  const float shared_p = m.misc->scalars[0];
#pragma unroll
  for (int k = 0; k < kPairsG; ++k) {
    const int p = m.gw + m.nw * k;
    if (p < pairs) {
      uint16_t y[2];
#pragma unroll
      for (int r = 0; r < 2; ++r) {
        Quad ga, ua;
        quad_zero(ga);
        quad_zero(ua);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (m.lane + 64 * j < quads) {
            const u32x4 xq = m.xn[m.lane + 64 * j];
            quad_acc(ga, xq, gv[k][r][j]);
            quad_acc(ua, xq, uv[k][r][j]);
          }
        const float gsum = quad_tree<64>(ga);
        const float usum = quad_tree<64>(ua);
        const int row = 2 * p + r;
        const float gb = rbf(gsum), ub = rbf(usum);
        const float activated = silu(gb);
        float out;
        if (row < routed) out = (activated * ub) * m.misc->probs[row / a.I];
        else out = rbf(rbf(activated) * ub) * shared_p;
        y[r] = f2bf(out);
      }
      if (m.lane == 0) word_store(Ly.x_active + p, pack_bf(y[0], y[1]), m.tag);
    }
  }
}

// ------------------------------------------ phase: MoE down + residual (S32)

// Per hidden row (moe.hex:371-434, simt_moe.hex:36-287): S32 over the
// concatenated routed activations (pair p reads expert ids[p / (I/2)]) and a
// separate S32 over the shared activations, one reference lane per physical
// lane (lanes 0-31 row 2w, lanes 32-63 row 2w+1);
// out = bf16(bf16(routed + residual) (+) bf16(shared)).
__device__ __forceinline__ void phase_down(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int H = a.H, half = m.lane >> 5, r32 = m.lane & 31;
  const int ip = a.I >> 1, rp = (a.K * a.I) >> 1, sp = a.SI >> 1;
  const int nj = (rp + 31) >> 5, nsj = (sp + 31) >> 5;
  const int prow = m.gw;
  const int row = 2 * prow + half;
  const bool has_rows = prow < (H >> 1);
  uint32_t wr[kDownJ], ws[kDownSJ];
  if (has_rows) {
    // pair p = r32 + 32j of the routed row lies in expert slot (32j) / ip when
    // ip is a multiple of 32 (host-checked), so the expert row base is
    // uniform per j; the lane offset selects the row (half) and the pair
#pragma unroll
    for (int j = 0; j < kDownJ; ++j) {
      if (j < nj) {
        const int slot = (32 * j) / ip;
        const int id = __builtin_amdgcn_readfirstlane(m.misc->ids[slot]);
        const uint16_t* w = Ly.down_exps + ((size_t)id * H + 2 * prow) * a.I;
        wr[j] = ldd_at(w, (uint32_t)(half * ip + min(r32 + 32 * j, rp - 1) - slot * ip) * 4u);
      }
    }
    const uint16_t* sw = Ly.sdown + (size_t)(2 * prow) * a.SI;
#pragma unroll
    for (int j = 0; j < kDownSJ; ++j)
      if (j < nsj) ws[j] = ldd_at(sw, (uint32_t)(half * sp + min(r32 + 32 * j, sp - 1)) * 4u);
  }
  poll_words<5>(m, Ly.x_active, rp + sp, Identity{}, m.vec);
  if (has_rows) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int j = 0; j < kDownJ; ++j) {
      const int p = r32 + 32 * j;
      if (j < nj && p < rp) pair_acc(lo, hi, m.vec[p], wr[j]);
    }
    const float routed_v = tree32_lanes(lo + hi);
    float slo = 0.0f, shi = 0.0f;
#pragma unroll
    for (int j = 0; j < kDownSJ; ++j) {
      const int p = r32 + 32 * j;
      if (j < nsj && p < sp) pair_acc(slo, shi, m.vec[rp + p], ws[j]);
    }
    const float shared_v = tree32_lanes(slo + shi);
    const uint16_t out = bf_add(f2bf(routed_v + bf2f(m.xa[row])), f2bf(shared_v));
    const uint16_t other = (uint16_t)__shfl_down((int)out, 32, 64);
    if (m.lane == 0) word_store(Ly.x_out + prow, pack_bf(out, other), m.tag);
  }
  __syncthreads();
}

// ------------------------------------- phase: attention scores (full layers)

// Every block normalises and rotates the query heads and the new key head
// (full_prepare.hex:3-82: head RMS with the adjacent-pair tree, neox RoPE on
// the first R channels), then scores its (KV head, key) items: 32-lane dots
// (lane l owns channels l, l+32, ..., serial from 0.0, then a 32-wide
// halving tree) for every query head of the group, x 1/sqrt(HD)
// (online.hex:4-18). The block that scores the new position writes K and V
// of that position into the cache; V is device-coherent and complete before
// that position's scores are published.
struct ScoreLds {
  float rope[256];
  float normed[kMW][256];
  uint16_t qhat[16 * 256];
  uint16_t khat[2 * 256];
};
static_assert(sizeof(ScoreLds) <= kLdsBigBytes, "score LDS");

__device__ __forceinline__ void phase_scores(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int HD = a.HD, Q = a.Q, KVH = a.KVH, hpk = Q / KVH;
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int64_t items = keys * KVH;
  ScoreLds* s = reinterpret_cast<ScoreLds*>(m.big);
  const int l32 = m.lane & 31, half = m.lane >> 5, kj = HD >> 5;
  // prefetch the cached keys of this block's first items
  const int64_t item0 = (int64_t)m.gw * 2 + half;
  float kv0[8];
  if (item0 < items) {
    const int kvh = (int)(item0 / keys);
    const int64_t key = item0 - (int64_t)kvh * keys;
    if (key < position) {
      const uint16_t* kr = a.cache + Ly.key_base + key * a.KVS + (int64_t)kvh * HD + l32;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < kj) kv0[j] = bf2f(G(kr)[32 * j]);
    }
  }
  // query parts of every head, then the raw key and value heads
  const int qwords = Q * (HD >> 1), kvwords = a.KVS >> 1;
  auto index = [&](int i) -> int {
    if (i < qwords) {
      const int hq = i / (HD >> 1), c = i - hq * (HD >> 1);
      return hq * HD + c;  // words of [q(HD) | gate(HD)] per head
    }
    return a.QS + (i - qwords);  // k words then v words
  };
  poll_words<5>(m, Ly.x_proj, qwords + 2 * kvwords, index, m.vec);
  const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
  const uint16_t* kraw = in16 + Q * HD;
  const uint16_t* vraw = kraw + a.KVS;
  // RoPE table for this position (rope.hex:5-17)
  const int rh = a.R >> 1;
  if (m.tid < rh) {
    float sn, cs;
    sincos_q((float)(uint32_t)position * G(a.freq)[m.tid], &sn, &cs);
    s->rope[m.tid] = cs;
    s->rope[rh + m.tid] = sn;
  }
  __syncthreads();
  // one wave per head: Q query heads then KVH key heads
  const int vpl = HD >> 6;  // values per lane (HD in {64, 128, 256})
  for (int h0 = 0; h0 < Q + KVH; h0 += kMW) {
    const int hh = h0 + m.wave;
    const bool is_q = hh < Q;
    float x[4], w[4];
    float t = 0.0f;
    if (hh < Q + KVH) {
      const uint16_t* src = is_q ? in16 + hh * HD : kraw + (hh - Q) * HD;
      const float* nw = is_q ? Ly.qnorm : Ly.knorm;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < vpl) {
          x[i] = bf2f(src[vpl * m.lane + i]);
          w[i] = G(nw)[vpl * m.lane + i];
        }
      // adjacent-pair tree: in-lane pairs first, then the lanes
      if (vpl == 1) t = x[0] * x[0];
      else if (vpl == 2) t = x[0] * x[0] + x[1] * x[1];
      else t = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
    }
    t = t + lane_down<1>(t);
    t = t + lane_down<2>(t);
    t = t + lane_down<4>(t);
    t = t + lane_down<8>(t);
    t = t + lane_down<16>(t);
    t = t + lane_down<32>(t);
    const float sum = __shfl(t, 0, 64);
    if (hh < Q + KVH) {
      const float inverse = 1.0f / nsqrt(sum / (float)HD + a.eps);
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (i < vpl) s->normed[m.wave][vpl * m.lane + i] = bf2f(bf_mul(f2bf(x[i] * inverse), f2bf(w[i])));
    }
    __syncthreads();
    if (hh < Q + KVH) {
      for (int c = m.lane; c < HD; c += 64) {
        const float nf = s->normed[m.wave][c];
        float result = nf;
        if (c < a.R) {
          const int pair = c % rh;
          const bool first = c < rh;
          const float partner = s->normed[m.wave][first ? pair + rh : pair];
          const float ac = nf * s->rope[pair];
          const float bs = partner * s->rope[pair + rh];
          result = first ? ac - bs : ac + bs;
        }
        const uint16_t rb = f2bf(result);
        if (is_q) s->qhat[hh * HD + c] = rb;
        else s->khat[(hh - Q) * HD + c] = rb;
      }
    }
    __syncthreads();
  }
  // score items: two per wave (32 lanes each)
  int round = 0;
  for (int64_t it = item0; it < items; it += 2 * (int64_t)m.nw, ++round) {
    const int kvh = (int)(it / keys);
    const int64_t key = it - (int64_t)kvh * keys;
    float kv[8];
    if (key == position) {
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < kj) kv[j] = bf2f(s->khat[kvh * HD + l32 + 32 * j]);
      // K and V of the new position into the cache (V device-coherent)
      uint16_t* kdst = a.cache + Ly.key_base + position * a.KVS + (int64_t)kvh * HD;
      uint16_t* vdst = a.cache + Ly.value_base + position * a.KVS + (int64_t)kvh * HD;
      for (int c = l32; c < HD; c += 32) {
        G(kdst)[c] = s->khat[kvh * HD + c];
        __hip_atomic_store(G(vdst) + c, vraw[kvh * HD + c], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else if (round == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) kv[j] = kv0[j];
    } else {
      const uint16_t* kr = a.cache + Ly.key_base + key * a.KVS + (int64_t)kvh * HD + l32;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < kj) kv[j] = bf2f(G(kr)[32 * j]);
    }
    for (int hq = 0; hq < hpk; ++hq) {
      const int head = kvh * hpk + hq;
      const uint16_t* qh = s->qhat + head * HD + l32;
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (j < kj) acc += bf2f(qh[32 * j]) * kv[j];
#pragma unroll
      for (int sh = 16; sh >= 1; sh >>= 1) acc += __shfl_down(acc, sh, 32);
      if (l32 == 0) word_store(Ly.x_scores + (size_t)head * a.cap + key, fbits(acc * a.attn_scale), m.tag);
    }
  }
  __syncthreads();
}

// ------------------------------------- phase: attention values (full layers)

// Per (query head, 16-channel chunk) item, the reference's online softmax in
// 8-key tiles (online.hex:272-331; per-kernel version attention.h): running
// maximum per tile as a prefix maximum of the tile maxima, alpha_t and
// p = exp(s - m_t) in parallel, then each channel's serial chain
// acc = acc * alpha_t + p_0 v_0 + ... + p_7 v_7 while lane 16 runs the
// denominator; out = bf16(bf16(acc / den) * sigmoid(gate)).
struct ValueLds {
  float p[kChunkKeys];
  float alpha[kChunkKeys / 8];
  u32x4 vs[kChunkKeys * 2];  // [key][16 channels] BF16
  float mx[1];               // tiles (the rest of the big area)
};
constexpr int kValueMxMax = (kLdsBigBytes - (int)offsetof(ValueLds, mx)) / 4;

__device__ __forceinline__ void phase_values(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int HD = a.HD, hpk = a.Q / a.KVH;
  const int chunks = HD / kValueChannels, items = a.Q * chunks;
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int tiles = (int)((keys + 7) >> 3);
  ValueLds* s = reinterpret_cast<ValueLds*>(m.big);
  const float ninf = bitsf(0xff800000u);
  for (int item = blockIdx.x; item < items; item += gridDim.x) {
    const int head = item / chunks, c0 = (item - head * chunks) * kValueChannels;
    const uint16_t* vbase = a.cache + Ly.value_base + (int64_t)(head / hpk) * HD + c0;
    // prefetch the first chunk's V rows (positions before the new one)
    u32x4 vpre[2];
    const int n0 = (int)min<int64_t>(kChunkKeys, (int64_t)tiles * 8);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int i = m.tid + kMT * j;
      const int64_t k = i >> 1;
      const int64_t safe = (k < keys && k != position) ? k : 0;
      if (i < 2 * n0) vpre[j] = G(reinterpret_cast<const u32x4*>(vbase + safe * a.KVS))[i & 1];
    }
    // scores of this head: poll every tile, keep the tile maxima
    const uint64_t* sc = Ly.x_scores + (size_t)head * a.cap;
    for (int t = m.tid; t < tiles; t += kMT) {
      float mt = ninf;
      uint64_t v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t k = (int64_t)t * 8 + j;
        v[j] = k < keys ? word_load(sc + k) : ((uint64_t)m.tag << 32);
      }
      unsigned spins = 0;
      while (true) {
        bool ready = true;
#pragma unroll
        for (int j = 0; j < 8; ++j) ready &= word_ready(v[j], m.tag);
        if (ready || spin_exhausted(m, spins)) break;
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (!word_ready(v[j], m.tag)) v[j] = word_load(sc + (int64_t)t * 8 + j);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t k = (int64_t)t * 8 + j;
        const float sk = bitsf((uint32_t)v[j]);
        mt = fmaxf(mt, k < keys ? sk : ninf);
        if (k < kChunkKeys) s->p[k] = sk;  // first chunk's scores, kept for the weights
      }
      s->mx[t] = mt;
    }
    // gate of this item's channels (word pairs)
    uint32_t gate_word = 0;
    if (m.tid < kValueChannels / 2)
      gate_word = poll_one(m, Ly.x_proj + ((head * 2 * HD + HD + c0) >> 1) + m.tid);
    __syncthreads();
    if (m.tid == 0) {
      float mm = ninf;
      for (int i = 0; i < tiles; ++i) {
        mm = fmaxf(mm, s->mx[i]);
        s->mx[i] = mm;
      }
    }
    __syncthreads();
    float acc = 0.0f, den = 0.0f;
    for (int64_t k0 = 0; k0 < (int64_t)tiles * 8; k0 += kChunkKeys) {
      const int n = (int)min<int64_t>(kChunkKeys, (int64_t)tiles * 8 - k0);  // multiple of 8
      // the new position's row is filled below by threads 0..15 (not staged here)
      if (k0 == 0) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int i = m.tid + kMT * j;
          if (i < 2 * n && (int64_t)(i >> 1) != position) s->vs[i] = vpre[j];
        }
      } else {
        for (int i = m.tid; i < 2 * n; i += kMT) {
          const int64_t k = k0 + (i >> 1);
          if (k == position) continue;
          const int64_t safe = k < keys ? k : 0;
          s->vs[i] = G(reinterpret_cast<const u32x4*>(vbase + safe * a.KVS))[i & 1];
        }
      }
      // the new position's V row was written in the previous phase
      if (position >= k0 && position < k0 + n && m.tid < kValueChannels) {
        const uint16_t v = __hip_atomic_load(G(vbase) + position * a.KVS + m.tid, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT);
        reinterpret_cast<uint16_t*>(s->vs)[(position - k0) * kValueChannels + m.tid] = v;
      }
      for (int i = m.tid; i < n; i += kMT) {
        const int64_t k = k0 + i;
        const float sk = k0 == 0 ? s->p[i] : bitsf((uint32_t)word_load(sc + k));
        s->p[i] = k < keys ? hexp(sk - s->mx[k >> 3]) : 0.0f;
      }
      for (int i = m.tid; i < n / 8; i += kMT) {
        const int tile = (int)(k0 / 8) + i;
        s->alpha[i] = hexp((tile > 0 ? s->mx[tile - 1] : ninf) - s->mx[tile]);
      }
      __syncthreads();
      if (m.wave == 0) {
        if (m.lane < kValueChannels) {
          const uint16_t* vh = reinterpret_cast<const uint16_t*>(s->vs) + m.lane;
          for (int i = 0; i < n / 8; ++i) {
            acc = acc * s->alpha[i];
#pragma unroll
            for (int j = 0; j < 8; ++j) acc = acc + s->p[i * 8 + j] * bf2f(vh[(i * 8 + j) * kValueChannels]);
          }
        } else if (m.lane == kValueChannels) {
          for (int i = 0; i < n / 8; ++i) {
            den = den * s->alpha[i];
#pragma unroll
            for (int j = 0; j < 8; ++j) den = den + s->p[i * 8 + j];
          }
        }
      }
      __syncthreads();
    }
    if (m.wave == 0) {
      den = __shfl(den, kValueChannels, 64);
      const uint32_t gw = __shfl((int)gate_word, m.lane >> 1, 64);
      const uint16_t gb = (m.lane & 1) ? (uint16_t)(gw >> 16) : (uint16_t)(gw & 0xffffu);
      uint16_t y = 0;
      if (m.lane < kValueChannels) y = f2bf(rbf(acc / den) * sigmoid(bf2f(gb)));
      const uint16_t other = (uint16_t)__shfl_down((int)y, 1, 64);
      if (m.lane < kValueChannels && (m.lane & 1) == 0)
        word_store(Ly.x_mix + ((head * HD + c0 + m.lane) >> 1), pack_bf(y, other), m.tag);
    }
    __syncthreads();
  }
}

// ------------------------------------------ phase: final norm + vocabulary

// output_norm, the S32 vocabulary GEMV (simt.hex:348-441) and the greedy
// first-index argmax (fused_argmax.hex) as a (value, lowest index) maximum.
// Eight lanes per row (lane q holds reference lanes 4q..4q+3), eight rows per
// wave per batch; a row streams in pieces of kVocabPiece quads per lane,
// double-buffered, so the accumulation stays in reference order.
constexpr int kVocabPiece = 8;

__device__ __forceinline__ void phase_head(const MegaArgs* pa, uint32_t tag) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaArgs& a = m.a;
  const int H = a.H, quads = H >> 3, V = a.V;
  const int q = m.lane & 7, g = m.lane >> 3;
  const int per_lane = quads >> 3;                                // quads per lane per row
  const int pieces = (per_lane + kVocabPiece - 1) / kVocabPiece;  // per row
  const int groups = (V + 7) / 8;  // 8-row groups; group gw + nw*b is this wave's batch b
  const int nbatches = m.gw < groups ? (groups - 1 - m.gw) / m.nw + 1 : 0;
  const int steps = nbatches * pieces;
  // piece t = (batch t / pieces, piece t % pieces); group base address is uniform
  auto load_piece = [&](u32x4* buf, int t) {
    const int b = t / pieces, pc = t - b * pieces;
    const int row0 = (m.gw + m.nw * b) * 8;
    const uint16_t* w = a.head + (size_t)row0 * H;
    const bool row_ok = row0 + g < V;
#pragma unroll
    for (int j = 0; j < kVocabPiece; ++j) {
      const int qi = q + 8 * (pc * kVocabPiece + j);
      if (row_ok && pc * kVocabPiece + j < per_lane)
        buf[j] = ldq_at(w, (uint32_t)g * (uint32_t)H * 2u + (uint32_t)qi * 16u);
    }
  };
  u32x4 b0[kVocabPiece], b1[kVocabPiece];
  if (steps > 0) load_piece(b0, 0);
  f32x4 w0, w1;
  norm_weights(m, a.out_norm, w0, w1);
  poll_words<2>(m, a.x_final, H >> 1, Identity{}, reinterpret_cast<uint32_t*>(m.xr));
  norm_row(m, m.xr, w0, w1);
  unsigned long long mine = 0ull;
  Quad acc;
  quad_zero(acc);
  auto consume = [&](const u32x4* buf, int t) {
    const int b = t / pieces, pc = t - b * pieces;
#pragma unroll
    for (int j = 0; j < kVocabPiece; ++j) {
      const int qi = q + 8 * (pc * kVocabPiece + j);
      if (pc * kVocabPiece + j < per_lane) quad_acc(acc, m.xn[qi], buf[j]);
    }
    if (pc == pieces - 1) {
      const float v = quad_tree<8>(acc);
      quad_zero(acc);
      const int row = (m.gw + m.nw * b) * 8 + g;
      if (q == 0 && row < V) {
        const uint16_t bb = f2bf(v);
        G(a.logits)[row] = bb;
        const unsigned long long key = logit_key(bb, (uint32_t)row);
        mine = key > mine ? key : mine;
      }
    }
  };
  for (int t = 0; t < steps; t += 2) {
    if (t + 1 < steps) load_piece(b1, t + 1);
    consume(b0, t);
    if (t + 1 < steps) {
      if (t + 2 < steps) load_piece(b0, t + 2);
      consume(b1, t + 1);
    }
  }
#pragma unroll
  for (int d = 32; d >= 8; d >>= 1) {
    const unsigned long long o = __shfl_down(mine, d, 64);
    mine = o > mine ? o : mine;
  }
  unsigned long long* wave_best = reinterpret_cast<unsigned long long*>(m.big);
  if (m.lane == 0) wave_best[m.wave] = mine;
  __syncthreads();
  if (m.tid == 0) {
    unsigned long long b = wave_best[0];
    for (int i = 1; i < kMW; ++i) b = wave_best[i] > b ? wave_best[i] : b;
    if (b) __hip_atomic_fetch_max(G(a.best), b, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// ------------------------------------------------------------- the kernel

__global__ __launch_bounds__(kMT) void k_decode_step(const MegaArgs* __restrict__ pa) {
  const uint32_t tag = (uint32_t)G(pa->params)[2];
  MegaMisc* misc = reinterpret_cast<MegaMisc*>(mega_lds + kLdsMisc);
  if (threadIdx.x == 0) {
    misc->abort = 0;
    if (blockIdx.x == 0) {
      // cleared before any output of this block exists, so before any block
      // can reach the head
      __hip_atomic_store(G(pa->best), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }
  __syncthreads();
  const int L = pa->L;
  const MegaLayer* layers = pa->layers;
  for (int l = 0; l < L; ++l) {
    const MegaLayer* ly = layers + l;
    phase_project(pa, tag, ly, l);
    const bool full = phase_ptr(ly)->full != 0;
    if (full) {
      phase_scores(pa, tag, ly);
      phase_values(pa, tag, ly);
    } else {
      phase_delta(pa, tag, ly);
      __syncthreads();
    }
    phase_outproj(pa, tag, ly, full ? phase_ptr(pa)->QS : phase_ptr(pa)->VS);
    phase_router(pa, tag, ly);
    phase_gate_up(pa, tag, ly);
    phase_down(pa, tag, ly);
  }
  phase_head(pa, tag);
}

}  // namespace cq35
