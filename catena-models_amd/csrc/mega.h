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
// raises the block's abort flag and the global error word (set to the step's
// tag), after which every wait of every block returns at once, so the grid
// always drains.
//
// Code size is a first-order cost here: the layer loop runs every phase once
// per layer, so the loop body must stay within the instruction cache. The
// kernel is therefore a template over the model shape (all widths
// compile-time constants, so loops have exact trip counts and no per-element
// guards), and the per-lane loads of a phase are straight-line code.
//
// Arithmetic and reduction orders are those of the per-kernel path
// (gemv.h, layers.h, attention.h), bit for bit.
#pragma once

#include <type_traits>

#include "attention.h"
#include "layers.h"

namespace cq35 {

constexpr int kMT = 512;       // threads per block
constexpr int kMW = kMT / 64;  // waves per block

// Per-wave work maxima.
constexpr int kPairsA = 3;       // projection row pairs per wave

// Model shapes the persistent step is compiled for. Widths follow
// ModelConfig (src/spec.rs:33-62); derived sizes as in spec.rs:293-362.
template <int H_, int V_, int Q_, int KVH_, int HD_, int R_, int KH_, int KD_, int VH_, int VD_,
          int E_, int K_, int I_, int SI_>
struct MegaShape {
  static constexpr int H = H_, V = V_, Q = Q_, KVH = KVH_, HD = HD_, R = R_, KH = KH_, KD = KD_,
                       VH = VH_, VD = VD_, E = E_, K = K_, I = I_, SI = SI_;
  static constexpr int KS = KH * KD, VS = VH * VD, QKV = 2 * KS + VS, QS = Q * HD, KVS = KVH * HD;
  static constexpr int QH = H / 8;            // BF16 quads per hidden row
  static constexpr int NQA = (QH + 63) / 64;  // S256 quads per lane per row
  static constexpr bool kDense = false;
  static_assert(H % 8 == 0 && H <= 2048, "hidden width");
  static_assert(KD % 32 == 0 && KD <= 128 && VD <= 128 && VD % 4 == 0, "DeltaNet head dims");
  static_assert(VH >= KH, "value heads");
  static_assert(HD == 64 || HD == 128 || HD == 256, "attention head dim");
  static_assert(QS <= 4096 && VS <= 4096 && KVS <= 512 && R <= 256 && R % 2 == 0, "attention widths");
  static_assert(QS / 2 + KVS <= 5 * kMT, "attention projection words");
  static_assert(E + 1 <= 1025 && K <= 64 && I % 64 == 0 && SI % 64 == 0, "expert shapes");
  static_assert((K * I + SI) / 2 + 1 <= 5 * kMT, "expert rows");
  static_assert(V % 8 == 0, "vocabulary in groups of 8 rows");
};
// qwen36-35b-a3b (src/spec.rs:153-183) and the two reduced MoE test shapes.
using Shape35BA3B = MegaShape<2048, 248320, 16, 2, 256, 64, 16, 128, 32, 128, 256, 8, 512, 512>;
using ShapeMiniMoE = MegaShape<512, 8192, 4, 2, 256, 64, 2, 128, 4, 128, 32, 8, 128, 256>;
using ShapeTinyMoE = MegaShape<256, 4096, 4, 1, 64, 16, 4, 32, 8, 32, 16, 4, 64, 128>;

struct MegaLayer {
  int full;
  const float* in_norm;
  const uint16_t* seg_w[4];
  int seg_rows[4];
  // linear (Gated DeltaNet)
  const uint16_t* alpha_w;  // ssm_alpha [VH, H]
  const uint16_t* beta_w;   // ssm_beta [VH, H]
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
  uint64_t* x_active;  // routed activations (K*I/2)
  uint64_t* x_shared;  // shared-expert bf16(bf16(silu(g)) * u), before the gate (SI/2)
  uint64_t* x_scores;  // Q * capacity F32 scores (full layers)
  uint64_t* x_out;     // output hidden row (H/2) = next layer's x_h
};

struct MegaArgs {
  const MegaLayer* layers;
  int L;
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
  int* ids_out;  // [L][K]: each layer's top-k expert ids of this step
  int64_t split_keys;  // values phase splits over more keys than this (0: never)
  uint64_t* trace;     // phase-trace builds: [grid][kTraceSlots] s_memrealtime stamps
};

// LDS carve-up (bytes); the "big" area is reused by the phases that need it.
constexpr int kLdsXn = 0;          // normalised input row, BF16 quads (H <= 2048)
constexpr int kLdsXr = 4096;       // raw hidden row (layer input; mixer residual)
constexpr int kLdsXa = 8192;       // raw post-mixer row (router input; FFN residual)
constexpr int kLdsVec = 12288;     // polled words (4096)
constexpr int kLdsMisc = 28672;    // logits, ids, probs, reductions
constexpr int kLdsBig = 36864;
constexpr int kLdsBigBytes = 53248;
constexpr int kMegaLdsBase = kLdsBig + kLdsBigBytes;

struct MegaMisc {
  float logits[1025];
  int ids[64];
  float probs[64];
  float chosen[64];
  float red[8];
  float scalars[8];
  int abort;
  int any_nan;
  int bid, grid;  // block index and grid size, re-read by every phase
  int tslot;      // phase-trace builds: the slot the current phase's poll stamps
  int tbase;      // phase-trace builds: the current layer's first slot
};
static_assert(sizeof(MegaMisc) <= kLdsBig - kLdsMisc, "misc LDS");

extern __shared__ __align__(16) unsigned char mega_lds[];

// ------------------------------------------------------------ phase trace
//
// Built with -DCQ35_PHASE_TRACE, every block records s_memrealtime (100 MHz)
// stamps in LDS and copies them to MegaArgs::trace at the end of the step:
// per layer l, for phase p (0 project, 1 delta or scores, 2 values,
// 3 output projection, 4 router, 5 gate/up, 6 down), slot
// l * kTraceLayerSlots + 2p holds the time its last wave finished the phase
// and 2p + 1 the time its inputs had all arrived (end of its poll); slots
// 14-17 hold the values phase's busy time per role (scan, products, channel
// chains, denominator chain) in 10 ns units (split-K: the flash phase's
// stages, 18 its items); slots 20-29 the last wave's time at points inside
// phases (kTraceMarks). Slot kTraceHead is the head's end, kTraceStart the
// step's start. Normal builds compile all of it away.
constexpr int kTraceLayerSlots = 32;
// Points inside phases (slot offsets in a layer).
enum TraceMark {
  kMarkProjectNormed = 20,  // project: input row polled and normalised
  kMarkDeltaConv = 21,      // delta: convolution done
  kMarkDeltaGates = 22,     // delta: L2 norms and gates done
  kMarkDeltaState = 23,     // delta: state update done
  kMarkRouterNormed = 24,   // router: post-mixer row normalised
  kMarkSelected = 25,       // gate/up: experts selected
  kMarkGateUpDone = 26,     // gate/up: outputs stored
  kMarkDownStaged = 27,     // down: staged weights and inputs in
  kMarkDownDone = 28,       // down: outputs stored
  kMarkOutprojDone = 29,    // output projection: outputs computed
};
constexpr int kTraceLayers = 48;
constexpr int kTraceHead = kTraceLayers * kTraceLayerSlots;
constexpr int kTraceStart = kTraceHead + 1;
constexpr int kTraceSlots = kTraceHead + 4;

__device__ __forceinline__ uint64_t* trace_lds();

__device__ __forceinline__ void trace_max(int slot) {
#ifdef CQ35_PHASE_TRACE
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_max(trace_lds() + slot, (uint64_t)__builtin_amdgcn_s_memrealtime(), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
#else
  (void)slot;
#endif
}

// The last wave's time at a point inside a phase of the current layer.
__device__ __forceinline__ void trace_mark(int mark) {
#ifdef CQ35_PHASE_TRACE
  trace_max(reinterpret_cast<volatile int*>(mega_lds + kLdsMisc + offsetof(MegaMisc, tbase))[0] + mark);
#else
  (void)mark;
#endif
}

__device__ __forceinline__ void trace_add(int slot, uint64_t v) {
#ifdef CQ35_PHASE_TRACE
  if ((threadIdx.x & 63) == 0)
    __hip_atomic_fetch_add(trace_lds() + slot, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#else
  (void)slot;
  (void)v;
#endif
}

// Busy time of one role loop: paused around each barrier.
struct RoleClock {
  uint64_t busy = 0, t0 = 0;
  __device__ __forceinline__ void resume() {
#ifdef CQ35_PHASE_TRACE
    t0 = __builtin_amdgcn_s_memrealtime();
#endif
  }
  __device__ __forceinline__ void pause() {
#ifdef CQ35_PHASE_TRACE
    busy += __builtin_amdgcn_s_memrealtime() - t0;
#endif
  }
};

// Pointers read from the argument tables are generic; every HBM access goes
// through the global address space so it compiles to global (not flat)
// memory instructions.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
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

// An opaque copy of a uniform pointer, kept in scalar registers: loads
// through it cannot be hoisted out of the phase that makes the copy, which
// keeps every phase's scalar state local to the phase. The tables are written
// by the host before the launch and never by the kernel, so they are read
// through the constant address space (scalar loads).
template <typename T>
__device__ __forceinline__ const CQ35_CONST T* phase_ptr(const T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  asm volatile("" : "+s"(lo), "+s"(hi));
  return (const CQ35_CONST T*)(((uint64_t)hi << 32) | lo);
}

// Per-thread view of one phase: the arguments, the step tag, thread
// coordinates and the LDS carve-up. Per-lane arithmetic is rebuilt in every
// phase instead of being hoisted out of the layer loop and held in registers
// across all phases.
struct Mega {
  const CQ35_CONST MegaArgs& a;
  uint32_t tag;
  // gw: global wave index, block-major (bid * kMW + wave); gs: the same
  // count interleaved across blocks (wave * grid + bid), so that a phase
  // whose last round covers only part of the waves spreads that round over
  // every CU instead of loading the first blocks with it
  int tid, lane, wave, gw, gs, nw, bid, grid;
  u32x4* xn;
  uint16_t* xr;
  uint16_t* xa;
  uint32_t* vec;
  MegaMisc* misc;
  unsigned char* big;
};

__device__ __forceinline__ Mega make_mega(const MegaArgs* pa, uint32_t tag) {
  const CQ35_CONST MegaArgs* a = phase_ptr(pa);
  int tid = threadIdx.x;
  asm volatile("" : "+v"(tid));
  // wave-level indices are uniform: scalar registers, so weight rows get
  // scalar base addresses (one 32-bit lane offset per load)
  // read from LDS (written once by the kernel), so values derived from the
  // block index are recomputed per phase rather than held across the loop
  const MegaMisc* mm = reinterpret_cast<const MegaMisc*>(mega_lds + kLdsMisc);
  const int bid = __builtin_amdgcn_readfirstlane(mm->bid);
  const int grid = __builtin_amdgcn_readfirstlane(mm->grid);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int gw = bid * kMW + wave;
  const int gs = wave * grid + bid;
  const int nw = grid * kMW;
  return Mega{*a,
              tag,
              tid,
              tid & 63,
              wave,
              gw,
              gs,
              nw,
              bid,
              grid,
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

// Spin bookkeeping of one polling loop: true when the wait must stop. The
// block's abort flag is checked every spin, the global error word and the
// spin limit every 256 spins. The error word holds the tag of the step that
// raised it, so an error left by an earlier step never stops a later one.
__device__ __forceinline__ bool spin_stop(const Mega& m, unsigned spins) {
  if (*abort_flag(m)) return true;
  if ((spins & 255u) != 0) return false;
  if (__hip_atomic_load(G(m.a.error), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == m.tag) {
    *abort_flag(m) = 1;
    return true;
  }
  if (spins > m.a.spin_limit) {
    __hip_atomic_store(G(m.a.error), m.tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *abort_flag(m) = 1;
    return true;
  }
  return false;
}

// Poll n words (word i at addr(i)) until every tag matches, then write the
// payloads to dst[i]. Up to MAXW words per thread; block-wide; ends with a
// barrier.
template <int MAXW, typename Addr>
__device__ __forceinline__ void poll_words(const Mega& m, int n, Addr addr, uint32_t* dst) {
  uint64_t v[MAXW];
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = min(m.tid + kMT * j, n - 1);
    v[j] = word_load(addr(i));
  }
  unsigned spins = 0;
  while (true) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) ready &= word_ready(v[j], m.tag);
    if (ready || spin_stop(m, ++spins)) break;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) {
      const int i = min(m.tid + kMT * j, n - 1);
      if (!word_ready(v[j], m.tag)) v[j] = word_load(addr(i));
    }
  }
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = m.tid + kMT * j;
    if (i < n) dst[i] = (uint32_t)v[j];
  }
  __syncthreads();
#ifdef CQ35_PHASE_TRACE
  trace_max(m.misc->tslot);
#endif
}

// poll_words for a word count far below MAXW * kMT: slots past n issue no
// load (in poll_words they re-read word n - 1, which with many slots makes
// every block hammer one line).
template <int MAXW, typename Addr>
__device__ __forceinline__ void poll_words_upto(const Mega& m, int n, Addr addr, uint32_t* dst) {
  uint64_t v[MAXW];
  const uint64_t done = (uint64_t)m.tag << 32;
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = m.tid + kMT * j;
    v[j] = i < n ? word_load(addr(i)) : done;
  }
  unsigned spins = 0;
  while (true) {
    bool ready = true;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) ready &= word_ready(v[j], m.tag);
    if (ready || spin_stop(m, ++spins)) break;
#pragma unroll
    for (int j = 0; j < MAXW; ++j) {
      const int i = m.tid + kMT * j;
      if (!word_ready(v[j], m.tag)) v[j] = word_load(addr(i));
    }
  }
#pragma unroll
  for (int j = 0; j < MAXW; ++j) {
    const int i = m.tid + kMT * j;
    if (i < n) dst[i] = (uint32_t)v[j];
  }
  __syncthreads();
#ifdef CQ35_PHASE_TRACE
  trace_max(m.misc->tslot);
#endif
}

// Words i of one buffer.
struct Span {
  const uint64_t* base;
  __device__ __forceinline__ const uint64_t* operator()(int i) const { return base + i; }
};

// Poll one word per calling thread (any subset of threads); returns the payload.
__device__ __forceinline__ uint32_t poll_one(const Mega& m, const uint64_t* p) {
  uint64_t v = word_load(p);
  unsigned spins = 0;
  while (!word_ready(v, m.tag) && !spin_stop(m, ++spins)) v = word_load(p);
  return (uint32_t)v;
}

// In-order sum of n floats in LDS (n a multiple of 4): every read is issued
// before the dependent adds, which keep the serial order.
template <int N>
__device__ __forceinline__ float serial_sum(const float* v) {
  static_assert(N % 4 == 0, "serial sum width");
  f32x4 x[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) x[i] = reinterpret_cast<const f32x4*>(v)[i];
  float total = 0.0f;
#pragma unroll
  for (int i = 0; i < N / 4; ++i) {
    total += x[i].x;
    total += x[i].y;
    total += x[i].z;
    total += x[i].w;
  }
  return total;
}

// ------------------------------------------------------- normalised input

// qwen35.normalize (qwen35.hex:912-977) of the raw row in `raw` into m.xn,
// with the norm weights prefetched by thread t < H/8 for octet t. The
// adjacent-pair tree over the padded width equals the octet tree, the 64-lane
// shuffle tree and ((w0 + w1) + (w2 + w3)) over waves 0-3 (threads past H/8
// hold +0, and joining a zero subtree is exact).
template <class S>
__device__ __forceinline__ void norm_row(const Mega& m, const uint16_t* raw, f32x4 w0, f32x4 w1,
                                         float eps) {
  const bool own = m.tid < S::QH;
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
  const float inverse = 1.0f / nsqrt(sum / (float)S::H + eps);
  if (own) m.xn[m.tid] = octet_scale(x, inverse, w0, w1);
  __syncthreads();
}

template <class S>
__device__ __forceinline__ void norm_weights(const Mega& m, const float* w, f32x4& w0, f32x4& w1) {
  const int o = min(m.tid, S::QH - 1);
  w0 = G(reinterpret_cast<const f32x4*>(w))[2 * o];
  w1 = G(reinterpret_cast<const f32x4*>(w))[2 * o + 1];
}

// Raw hidden row of layer l into `raw`: the embedding row for layer 0,
// otherwise the previous layer's output words.
template <class S>
__device__ __forceinline__ void load_hidden(const Mega& m, const uint64_t* words, uint16_t* raw,
                                            bool embedding) {
  if (embedding) {
    const uint64_t token = G(m.a.params)[1];
    const u32x4* row = reinterpret_cast<const u32x4*>(m.a.embed + token * (uint64_t)S::H);
    if (m.tid < S::QH) reinterpret_cast<u32x4*>(raw)[m.tid] = G(row)[m.tid];
    __syncthreads();
  } else {
    poll_words<(S::H / 2 + kMT - 1) / kMT>(m, S::H / 2, Span{words}, reinterpret_cast<uint32_t*>(raw));
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

// pair_acc over j = 0 .. NJ-1 with x[32 j] and w[32 j] in LDS, in order. The
// reads of a batch are issued before the products of the previous one (the
// scheduler otherwise waits out one LDS round trip per pair of reads).
template <int NJ>
__device__ __forceinline__ void pair_chain_lds(float& lo, float& hi, const uint32_t* x, const CQ35_LDS uint32_t* w) {
  constexpr int B = NJ < 8 ? NJ : 8, NB = NJ / B;
  static_assert(NJ % B == 0, "pair chain batches");
  uint32_t xv[2][B], wv[2][B];
#pragma unroll
  for (int i = 0; i < B; ++i) {
    xv[0][i] = x[32 * i];
    wv[0][i] = w[32 * i];
  }
#pragma unroll
  for (int b = 0; b < NB; ++b) {
    if (b + 1 < NB) {
#pragma unroll
      for (int i = 0; i < B; ++i) {
        xv[(b + 1) & 1][i] = x[32 * ((b + 1) * B + i)];
        wv[(b + 1) & 1][i] = w[32 * ((b + 1) * B + i)];
      }
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int i = 0; i < B; ++i) pair_acc(lo, hi, xv[b & 1][i], wv[b & 1][i]);
    __builtin_amdgcn_sched_barrier(0);
  }
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
// reference lanes 4q..4q+3; row pairs (2p, 2p+1) per output word. The
// weights are issued by the previous phase (the last phase of the previous
// layer), so they stream while that phase computes.
// Pairs k < kPairsEarly are issued one phase early (before the previous
// layer's down projection waits); the rest at the start of the projection.
constexpr int kPairsEarly = 2;
template <class S>
struct ProjRegs {
  u32x4 w[kPairsA][2][S::NQA];
};

// Row pairs of the projection phase: every row of a full layer; of a
// linear layer the q | k | v rows only (the z rows, needed only by the gated
// norm at the end of the delta phase, are computed during that phase by the
// blocks that have no value head: project_z).
template <class S>
__device__ __forceinline__ int project_pairs(const CQ35_CONST MegaLayer& Ly) {
  return Ly.full ? (Ly.seg_rows[0] + Ly.seg_rows[1] + Ly.seg_rows[2] + Ly.seg_rows[3]) >> 1 : S::QKV / 2;
}

template <class S, int K0, int K1>
__device__ __forceinline__ void issue_project(const MegaArgs* pa, const MegaLayer* ly, ProjRegs<S>& r) {
  const Mega m = make_mega(pa, 0);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const int pairs = project_pairs<S>(Ly);
#pragma unroll
  for (int k = K0; k < K1; ++k) {
    const int p = m.gs + m.nw * k;
    if (p < pairs) {
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const uint16_t* w = seg_row(Ly, 2 * p + rr, S::H);
#pragma unroll
        for (int j = 0; j < S::NQA; ++j)
          r.w[k][rr][j] = ldq_at(w, (uint32_t)min(m.lane + 64 * j, S::QH - 1) * 16u);
      }
    } else {
      // defined on every path, so the registers are not carried across phases
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int j = 0; j < S::NQA; ++j) r.w[k][rr][j] = u32x4{0u, 0u, 0u, 0u};
    }
  }
}

template <class S>
__device__ __forceinline__ void phase_project(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int l,
                                              ProjRegs<S>& r) {
  issue_project<S, kPairsEarly, kPairsA>(pa, ly, r);
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  constexpr int NQ = S::NQA;
  const int pairs = project_pairs<S>(Ly);
  f32x4 w0, w1;
  norm_weights<S>(m, Ly.in_norm, w0, w1);
  load_hidden<S>(m, Ly.x_h, m.xr, l == 0);
  norm_row<S>(m, m.xr, w0, w1, m.a.eps);
  trace_mark(kMarkProjectNormed);
  // this lane's input quads, unpacked once for all its rows
  float xl[NQ][4], xh[NQ][4];
#pragma unroll
  for (int j = 0; j < NQ; ++j) {
    const u32x4 xq = (S::QH % 64 == 0 || m.lane + 64 * j < S::QH) ? m.xn[m.lane + 64 * j] : u32x4{0u, 0u, 0u, 0u};
    quad_unpack(xq, xl[j], xh[j]);
  }
#pragma unroll
  for (int k = 0; k < kPairsA; ++k) {
    const int p = m.gs + m.nw * k;
    if (p < pairs) {
      Quad acc[2];
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        quad_zero(acc[rr]);
#pragma unroll
        for (int j = 0; j < NQ; ++j)
          if (S::QH % 64 == 0 || m.lane + 64 * j < S::QH) quad_acc_f(acc[rr], xl[j], xh[j], r.w[k][rr][j]);
      }
      const float v = quad_tree64_pair_end(acc[0], acc[1]);  // row 2p in lane 31, 2p + 1 in lane 63
      const float v0 = lane_value(v, 31), v1 = lane_value(v, 63);
      if (m.lane == 0) word_store(Ly.x_proj + p, pack_bf(f2bf(v0), f2bf(v1)), m.tag);
    }
  }
}

// ------------------------------------------- phase: Gated DeltaNet (linear)

// One block per value head h (key head h % KH): the 4-tap convolution of the
// head's q, k and v channels (linear_prepare.hex:2-64), serial L2 norms of q
// and k (linear_prepare.hex:84-131), the gates (fused_delta.hex:1-20), the
// delta step of the head's VD channels with the state staged in LDS
// (cached_delta.hex:69-168, D32 trees) and the gated RMSNorm x SiLU(z)
// (cooperative_norm.hex:139-182). The head's alpha and beta rows of the
// grouped projection (S256 over the normalised row the block already holds)
// are computed here by waves 0 and 1. The v channels' conv history is written
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
  float gates[4];       // decay, rate, norms
  uint16_t ab[2];       // alpha, beta of the head
};
static_assert(sizeof(DeltaLds) <= kLdsBigBytes, "delta LDS");

// The z rows of a linear layer's grouped projection (rows QKV .. QKV + VS,
// pair words QKV/2 + zp), on the blocks that have no value head, while the
// value-head blocks run the delta step: the same S256 rows and words as the
// projection phase (group_projection.hex:3-97), over the normalised row the
// block still holds from that phase. Worker w (interleaved across the
// worker blocks) takes pairs w, w + W, ...
template <class S>
__device__ __forceinline__ void project_z(const Mega& m, const CQ35_CONST MegaLayer& Ly) {
  constexpr int ZP = S::VS / 2, NQ = S::NQA;
  const int workers = (m.grid - S::VH) * kMW;
  const int w0 = m.wave * (m.grid - S::VH) + (m.bid - S::VH);
  float xl[NQ][4], xh[NQ][4];
  bool unpacked = false;
  for (int z0 = w0; z0 < ZP; z0 += 2 * workers) {
    // two pairs' rows in flight
    u32x4 wv[2][2][NQ];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int zp = min(z0 + k * workers, ZP - 1);
#pragma unroll
      for (int rr = 0; rr < 2; ++rr) {
        const uint16_t* w = seg_row(Ly, S::QKV + 2 * zp + rr, S::H);
#pragma unroll
        for (int j = 0; j < NQ; ++j) wv[k][rr][j] = ldq_at(w, (uint32_t)min(m.lane + 64 * j, S::QH - 1) * 16u);
      }
    }
    if (!unpacked) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const u32x4 xq = (S::QH % 64 == 0 || m.lane + 64 * j < S::QH) ? m.xn[m.lane + 64 * j] : u32x4{0u, 0u, 0u, 0u};
        quad_unpack(xq, xl[j], xh[j]);
      }
      unpacked = true;
    }
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int zp = z0 + k * workers;
      if (zp < ZP) {
        Quad acc[2];
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
          quad_zero(acc[rr]);
#pragma unroll
          for (int j = 0; j < NQ; ++j)
            if (S::QH % 64 == 0 || m.lane + 64 * j < S::QH) quad_acc_f(acc[rr], xl[j], xh[j], wv[k][rr][j]);
        }
        const float v = quad_tree64_pair_end(acc[0], acc[1]);  // row 2zp in lane 31, 2zp + 1 in lane 63
        const float v0 = lane_value(v, 31), v1 = lane_value(v, 63);
        if (m.lane == 0) word_store(Ly.x_proj + S::QKV / 2 + zp, pack_bf(f2bf(v0), f2bf(v1)), m.tag);
      }
    }
  }
}

template <class S>
__device__ __forceinline__ void phase_delta(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  const int h = m.bid;
  if (h >= S::VH) {  // uniform per block
    if constexpr (!S::kDense) project_z<S>(m, Ly);
    return;
  }
  constexpr int KD = S::KD, VD = S::VD, NCH = 2 * KD + VD;
  constexpr int KJ = KD / 32, CPP = kMT / 8, PASSES = (VD + CPP - 1) / CPP;
  static_assert(NCH <= kMT, "delta shape");
  const int kh = h % S::KH;
  DeltaLds* d = reinterpret_cast<DeltaLds*>(m.big);
  uint16_t* st_g = a.cache + Ly.state_base + (size_t)h * VD * KD;
  // prefetch: this thread's state slices (channel c = pass * CPP + tid / 8,
  // key elements 4q + i + 32j, 8 bytes per j), conv taps, history, gates
  const int q = m.lane & 7, sub = m.tid >> 3;
  u32x2 sv[PASSES][KJ];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int cc = min(ps * CPP + sub, VD - 1);
#pragma unroll
    for (int j = 0; j < KJ; ++j)
      sv[ps][j] = *G(reinterpret_cast<const u32x2*>(st_g + (size_t)cc * KD + 4 * q + 32 * j));
  }
  const int64_t position = (int64_t)G(a.params)[0];
  int ch = 0;
  if (m.tid < KD) ch = kh * KD + m.tid;
  else if (m.tid < 2 * KD) ch = S::KS + kh * KD + (m.tid - KD);
  else ch = 2 * S::KS + h * VD + (m.tid - 2 * KD);
  const bool conv_thread = m.tid < NCH;
  f32x4 taps_w = {0.f, 0.f, 0.f, 0.f};
  float hist[3] = {0.f, 0.f, 0.f};
  const uint16_t* history = a.cache + Ly.conv_base;
  if (conv_thread) {
    taps_w = G(reinterpret_cast<const f32x4*>(Ly.conv_w))[ch];
#pragma unroll
    for (int k = 0; k < 3; ++k) hist[k] = bf2f(G(history)[((position + k) % 3) * S::QKV + ch]);
  }
  const float dt = G(Ly.dt)[h], aa = G(Ly.a)[h];
  const float gw = m.tid < VD ? G(Ly.gnorm)[m.tid] : 0.0f;
  // alpha (wave kMW - 2) and beta (wave kMW - 1) rows of head h, on the
  // waves that have no convolution channel (MoE shapes: S256 here; dense
  // shapes: S32 rows of the projection phase)
  static_assert(NCH <= kMT - 128, "alpha/beta waves");
  constexpr int kAB = kMW - 2;
  u32x4 abw[S::NQA];
  if (!S::kDense && m.wave >= kAB) {
    const uint16_t* w = (m.wave == kAB ? Ly.alpha_w : Ly.beta_w) + (size_t)h * S::H;
#pragma unroll
    for (int j = 0; j < S::NQA; ++j) abw[j] = ldq_at(w, (uint32_t)min(m.lane + 64 * j, S::QH - 1) * 16u);
  }
  // inputs: q | k | v of this head, z (projection words; MoE shapes: z is
  // polled before the gated norm, its rows being computed meanwhile)
  constexpr int qw = KD / 2, vw = VD / 2;
  constexpr int zbase = S::QKV;
  constexpr int nwords = 2 * qw + vw + (S::kDense ? vw + 2 : 0);
  const uint64_t* proj = Ly.x_proj;
  auto addr = [&](int i) -> const uint64_t* {
    if (i < qw) return proj + ((kh * KD) >> 1) + i;
    if (i < 2 * qw) return proj + ((S::KS + kh * KD) >> 1) + (i - qw);
    if (i < 2 * qw + vw) return proj + ((2 * S::KS + h * VD) >> 1) + (i - 2 * qw);
    if (i < 2 * qw + 2 * vw) return proj + ((zbase + h * VD) >> 1) + (i - 2 * qw - vw);
    // dense: the words holding alpha row QKV + VS + h and beta row QKV + VS + VH + h
    return proj + ((S::QKV + S::VS + (i - 2 * qw - 2 * vw) * S::VH + h) >> 1);
  };
  static_assert(S::kDense || nwords == 2 * qw + vw, "z words polled later");
  poll_words<(nwords + kMT - 1) / kMT>(m, nwords, addr, m.vec);
  if constexpr (S::kDense) {
    static_assert(S::VH % 2 == 0, "alpha and beta rows share a word's parity");
    if (m.tid < 2) {
      const uint32_t w = m.vec[2 * qw + 2 * vw + m.tid];
      d->ab[m.tid] = (uint16_t)((h & 1) ? (w >> 16) : (w & 0xffffu));
    }
  } else if (m.wave >= kAB) {
    Quad acc;
    quad_zero(acc);
#pragma unroll
    for (int j = 0; j < S::NQA; ++j)
      if (S::QH % 64 == 0 || m.lane + 64 * j < S::QH) quad_acc(acc, m.xn[m.lane + 64 * j], abw[j]);
    const float v = quad_tree<64>(acc);
    if (m.lane == 0) d->ab[m.wave - kAB] = f2bf(v);
  }
  const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
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
      G(a.cache)[Ly.conv_base + (position % 3) * S::QKV + ch] = current;
    }
  }
  __syncthreads();
  trace_mark(kMarkDeltaConv);
  // serial L2 sums (q: thread 0, k: thread 64) and the gates (thread 128)
  if (m.tid == 0 || m.tid == 64) {
    const float total = serial_sum<KD>(d->sq + (m.tid == 0 ? 0 : KD));
    d->gates[2 + (m.tid == 0 ? 0 : 1)] = nsqrt(total + bitsf(0x358637bdu));
  } else if (m.tid == 128) {
    const uint16_t alpha = d->ab[0];
    const uint16_t beta = d->ab[1];
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
  trace_mark(kMarkDeltaGates);
  // delta step: 64 channels per pass, 8 lanes per channel; lane q holds the
  // D32 reference lanes 4q..4q+3, i.e. key elements 4q + i + 32j (i, j < 4):
  // per i a serial chain over j from 0.0, then the 32-lane halving tree
  // (strides 16, 8, 4 across lanes, 2 and 1 in-lane; tree_levels order).
  // The state stays in registers and is written back from them.
  const float decay = d->gates[0], rate = d->gates[1];
  float kv[KJ][4], qv[KJ][4];
#pragma unroll
  for (int j = 0; j < KJ; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[j][i] = bf2f(d->khat[4 * q + i + 32 * j]);
      qv[j][i] = bf2f(d->qhat[4 * q + i + 32 * j]);
    }
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int c = ps * CPP + sub;
    const bool valid = c < VD;
    const int cc = valid ? c : 0;
    float old[KJ][4];
    float v[4];
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      old[j][0] = lo2f(sv[ps][j].x); old[j][1] = hi2f(sv[ps][j].x);
      old[j][2] = lo2f(sv[ps][j].y); old[j][3] = hi2f(sv[ps][j].y);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float acc = 0.0f;
#pragma unroll
      for (int j = 0; j < KJ; ++j) acc += old[j][i] * kv[j][i];
      v[i] = acc;
    }
    tree_levels<8>(v[0], v[1], v[2], v[3]);
    float total = (v[0] + v[2]) + (v[1] + v[3]);
    // the group's first lane holds the tree value: broadcast within the 8 lanes
    total = __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, total), 0x18));
    const float value = d->conv[2 * KD + cc];
    const float delta = (value - total * decay) * rate;
    float w[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < KJ; ++j) {
      float nx[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        nx[i] = old[j][i] * decay + kv[j][i] * delta;
        w[i] += nx[i] * qv[j][i];
      }
      if (valid)
        *G(reinterpret_cast<u32x2*>(st_g + (size_t)c * KD + 4 * q + 32 * j)) =
            u32x2{pack_bf(f2bf(nx[0]), f2bf(nx[1])), pack_bf(f2bf(nx[2]), f2bf(nx[3]))};
    }
    tree_levels<8>(w[0], w[1], w[2], w[3]);
    const float out = (w[0] + w[2]) + (w[1] + w[3]);
    if (q == 0 && valid) d->core[c] = f2bf(out * a.delta_scale);
  }
  __syncthreads();
  trace_mark(kMarkDeltaState);
  if constexpr (!S::kDense) {
    // the head's z words (computed by the blocks without a value head)
    if (m.tid < vw) m.vec[2 * qw + vw + m.tid] = poll_one(m, addr(2 * qw + vw + m.tid));
  }
  // gated RMSNorm with a serial sum (cooperative_norm.hex:139-182)
  if (m.tid < VD) {
    const float v = bf2f(d->core[m.tid]);
    d->sq[m.tid] = v * v;
  }
  __syncthreads();
  if (m.tid == 0) d->gates[2] = serial_sum<VD>(d->sq);
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
// simt.hex:442-538) over the polled mixer output (COLS BF16): one row per
// wave and all waves of every block; physical lane = reference lane l, which
// visits pairs l, l+64, ... (one dword each, 256 contiguous bytes per wave),
// then the 64-lane tree. Waves 2i and 2i+1 take rows 2p and 2p+1,
// p = block + grid * i, and the even wave stores the word. Blocks kh < KH of a
// linear layer also write the q and k conv history of key head kh.
// With kDown (dense SwiGLU down projection, the same S64 order): input the
// gate/up activations x_active (I BF16), weights sdown, residual the
// post-mixer row, output x_out.
template <class S, int COLS, bool kDown = false>
__device__ __forceinline__ void phase_outproj(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int NP = COLS / 2, NJ = NP / 64;
  static_assert(NP % 64 == 0 && NP <= 4096, "output projection width");
  const int p = m.bid + m.grid * (m.wave >> 1);
  const int row = 2 * p + (m.wave & 1);
  const bool has_row = p < S::H / 2;
  uint32_t wv[NJ];
  if (has_row) {
    const uint16_t* w = (kDown ? Ly.sdown : Ly.out_w) + (size_t)row * COLS;
#pragma unroll
    for (int j = 0; j < NJ; ++j) wv[j] = ldd_at(w, (uint32_t)(m.lane + 64 * j) * 4u);
  }
  poll_words<(NP + kMT - 1) / kMT>(m, NP, Span{kDown ? Ly.x_active : Ly.x_mix}, m.vec);
  if (!kDown && !Ly.full && m.bid < S::KH) {
    // q and k history of key head kh = the block index (its raw values are
    // still in this block's LDS from the previous phase).
    const DeltaLds* d = reinterpret_cast<const DeltaLds*>(m.big);
    const int kh = m.bid;
    const int64_t slot = ((int64_t)G(a.params)[0] % 3) * S::QKV;
    if (m.tid < 2 * S::KD) {
      const int ch = m.tid < S::KD ? kh * S::KD + m.tid : S::KS + kh * S::KD + (m.tid - S::KD);
      G(a.cache)[Ly.conv_base + slot + ch] = d->raw_qk[m.tid];
    }
  }
  uint16_t o = 0;
  if (has_row) {
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) pair_acc(lo, hi, m.vec[m.lane + 64 * j], wv[j]);
    const float v = tree64_lanes(lo + hi);
    o = bf_add(f2bf(v), kDown ? m.xa[row] : m.xr[row]);
    if (m.lane == 0 && (m.wave & 1)) m.misc->red[4 + (m.wave >> 1)] = __builtin_bit_cast(float, (uint32_t)o);
  }
  if (!kDown) trace_mark(kMarkOutprojDone);
  __syncthreads();
  if (has_row && m.lane == 0 && !(m.wave & 1)) {
    const uint16_t other = (uint16_t)__builtin_bit_cast(uint32_t, m.misc->red[4 + (m.wave >> 1)]);
    word_store((kDown ? Ly.x_out : Ly.x_attn) + p, pack_bf(o, other), m.tag);
  }
}

// ----------------------------------------------- phase: MoE router (S32 F32)

// Every block normalises the post-mixer row (post_attention_norm) into m.xn
// for the router and the gate/up phase and keeps the raw row for the FFN
// residual. Even waves 2i compute router row block + grid * i (rows
// [0, E] spread one per block; moe.hex:4-84): physical lane 2r + h runs
// reference lanes r's low (h = 0) or high (h = 1) accumulator over floats
// 64k + lane. The four odd waves of block b compute the shared expert's
// gate/up rows of pair b (dual S256, moe.hex:254-333), one row each (gate
// 2b, up 2b, gate 2b+1, up 2b+1), and wave 1 combines them up to the
// routing-dependent factor: t = bf16(bf16(silu(bf16 g)) * bf16 u); the down
// phase applies bf16(t * sigmoid(shared logit)), the same roundings as the
// reference.
template <class S>
__device__ __forceinline__ void phase_router(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  constexpr int H = S::H, QH = S::QH, NQ = S::NQA, ROWS = S::E + 1, NJ = (H + 63) / 64;
  static_assert(S::SI / 2 <= 256, "shared pairs");
  float wv[NJ];
  u32x4 sv[NQ];
  const int rrow = m.bid + m.grid * (m.wave >> 1);  // router row of an even wave
  const int sp = m.bid;                              // shared pair of the odd waves
  const int role = m.wave >> 1;                      // odd waves: gate 2sp, up 2sp, gate 2sp+1, up 2sp+1
  const bool router_wave = !(m.wave & 1) && rrow < ROWS;
  const bool shared_wave = (m.wave & 1) && sp < S::SI / 2;
  if (router_wave) {
    const float* w = rrow < S::E ? Ly.router + (size_t)rrow * H : Ly.shared_gate;
#pragma unroll
    for (int j = 0; j < NJ; ++j) wv[j] = ldf_at(w, (uint32_t)min(64 * j + m.lane, H - 1) * 4u);
  } else if (shared_wave) {
    const uint16_t* w = ((role & 1) ? Ly.sup : Ly.sgate) + (size_t)(2 * sp + (role >> 1)) * H;
#pragma unroll
    for (int j = 0; j < NQ; ++j) sv[j] = ldq_at(w, (uint32_t)min(m.lane + 64 * j, QH - 1) * 16u);
  }
  f32x4 w0, w1;
  norm_weights<S>(m, Ly.post_norm, w0, w1);
  poll_words<(H / 2 + kMT - 1) / kMT>(m, H / 2, Span{Ly.x_attn}, reinterpret_cast<uint32_t*>(m.xa));
  norm_row<S>(m, m.xa, w0, w1, m.a.eps);
  trace_mark(kMarkRouterNormed);
  if (router_wave) {
    const uint16_t* xe = reinterpret_cast<const uint16_t*>(m.xn);
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NJ; ++j)
      if (H % 64 == 0 || 64 * j + m.lane < H) acc += bf2f(xe[64 * j + m.lane]) * wv[j];
    float v = acc + lane_down<1>(acc);
    v += lane_down<32>(v);
    v += lane_down<16>(v);
    v += lane_down<8>(v);
    v += lane_down<4>(v);
    v += lane_down<2>(v);
    if (m.lane == 0) word_store(Ly.x_router + rrow, fbits(v), m.tag);
  } else if (shared_wave) {
    Quad acc;
    quad_zero(acc);
#pragma unroll
    for (int j = 0; j < NQ; ++j)
      if (QH % 64 == 0 || m.lane + 64 * j < QH) quad_acc(acc, m.xn[m.lane + 64 * j], sv[j]);
    const float v = rbf(quad_tree<64>(acc));
    if (m.lane == 0) m.misc->scalars[role] = v;
  }
  __syncthreads();
  if (m.wave == 1 && m.lane == 0 && sp < S::SI / 2) {
    uint16_t t[2];
#pragma unroll
    for (int r = 0; r < 2; ++r) t[r] = f2bf(rbf(silu(m.misc->scalars[2 * r])) * m.misc->scalars[2 * r + 1]);
    word_store(Ly.x_shared + sp, pack_bf(t[0], t[1]), m.tag);
  }
}

// ----------------------------------------- phase: top-k select + gate / up

// Every block ranks the experts itself (moe.hex:86-252). The reference's
// rank is rank(e) = #{i : l_i > l_e} + #{i < e : !(l_e > l_i)}, ids[rank] = e
// for rank < K. Without NaNs this is the descending order with ties to the
// lower index, so wave 0 takes K rounds: the wave-wide maximum of the
// order-preserving integer images of the logits (+0 and -0 equal), then the
// lowest expert index holding it (ballots over the lanes' candidate groups,
// lane l holding experts l + 64c). With a NaN the formula is evaluated
// directly. Then p_j = exp(l_j - l_0) / den with den summed left to right.
__device__ __forceinline__ uint32_t logit_order(float le) {
  const uint32_t u = le == 0.0f ? 0u : fbits(le);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);  // >= 0x00800000 for non-NaN
}

template <int S>
__device__ __forceinline__ uint32_t umax_down(uint32_t v) {
  const uint32_t o = __builtin_bit_cast(uint32_t, lane_down<S>(__builtin_bit_cast(float, v)));
  return o > v ? o : v;
}

template <class S>
__device__ __forceinline__ void select_experts(const Mega& m) {
  MegaMisc* s = m.misc;
  static_assert(S::E <= 64 * 64 && S::K <= 64, "expert count");
  constexpr int PER = (S::E + 63) / 64;  // candidates per lane
  if (m.wave == 0) {
    uint32_t ov[PER];  // 0: absent or taken (below every non-NaN image)
    bool nan = false;
#pragma unroll
    for (int c = 0; c < PER; ++c) {
      const int e = m.lane + 64 * c;
      ov[c] = 0u;
      if (e < S::E) {
        const float le = s->logits[e];
        nan |= le != le;
        ov[c] = logit_order(le);
      }
    }
    const bool any_nan = __any(nan);
    if (!any_nan) {
      for (int k = 0; k < S::K; ++k) {
        uint32_t best = ov[0];
#pragma unroll
        for (int c = 1; c < PER; ++c) best = ov[c] > best ? ov[c] : best;
        best = umax_down<32>(best);
        best = umax_down<16>(best);
        best = umax_down<8>(best);
        best = umax_down<4>(best);
        best = umax_down<2>(best);
        best = umax_down<1>(best);
        const uint32_t win = __builtin_amdgcn_readfirstlane(best);
        int e = S::E;
#pragma unroll
        for (int c = PER - 1; c >= 0; --c) {
          const unsigned long long hit = __ballot(ov[c] == win);
          if (hit) e = 64 * c + __builtin_ctzll(hit);
        }
#pragma unroll
        for (int c = 0; c < PER; ++c)
          if (64 * c + m.lane == e) ov[c] = 0u;  // taken
        if (m.lane == 0) s->ids[k] = e;
      }
      // probabilities right here: lane j < K holds l_j
      const float lj = m.lane < S::K ? s->logits[s->ids[m.lane]] : 0.0f;
      const float l0 = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, lj)));
      const float ex = m.lane < S::K ? hexp(lj - l0) : 0.0f;
      float den = 0.0f;
#pragma unroll
      for (int j = 0; j < S::K; ++j)
        den = den + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ex), j));
      if (m.lane < S::K) s->probs[m.lane] = ex / den;
    }
    if (m.lane == 0) s->any_nan = any_nan ? 1 : 0;
  }
  __syncthreads();
  if (s->any_nan) {
    // NaNs can make two experts share a rank and leave another unassigned:
    // the largest expert index of a shared rank takes it (the restatement's
    // ascending scatter, deterministic here through an LDS maximum), and an
    // unassigned rank k keeps expert k (as the batched select does)
    if (m.tid < S::K) s->ids[m.tid] = -1;
    __syncthreads();
    for (int e = m.tid; e < S::E; e += kMT) {
      const float le = s->logits[e];
      int rank = 0;
      for (int i = 0; i < S::E; ++i) {
        const float o = s->logits[i];
        rank += (o > le) ? 1 : ((i < e && !(le > o)) ? 1 : 0);
      }
      if (rank < S::K) atomicMax(&s->ids[rank], e);
    }
    __syncthreads();
    if (m.tid < S::K) {
      const int e = s->ids[m.tid] >= 0 ? s->ids[m.tid] : m.tid;
      s->ids[m.tid] = e;
      s->chosen[m.tid] = s->logits[e];
    }
    __syncthreads();
    if (m.wave == 0) {
      const float ex = m.lane < S::K ? hexp(s->chosen[m.lane] - s->chosen[0]) : 0.0f;
      float den = 0.0f;
      for (int j = 0; j < S::K; ++j) den = den + __shfl(ex, j, 64);
      if (m.lane < S::K) s->probs[m.lane] = ex / den;
    }
    __syncthreads();
  }
}

// Down-projection weights, staged in LDS by DMA (global_load_lds, 16 bytes
// per lane) as soon as the experts are known, so no registers hold them and
// one instruction moves 1 KB. Waves 0-3 of every block own one row pair
// each, prow = block + grid * wave; per wave the staging is
//   [row A routed RP][32][row B routed RP][row A shared SP][32][row B shared SP]
// dwords (the pads keep the two rows on different LDS banks).
template <class S>
struct DownLayout {
  static constexpr int RP = S::K * S::I / 2, SP = S::SI / 2, IP = S::I / 2;
  static constexpr int A_R = 0, B_R = RP + 32, A_S = 2 * RP + 32, B_S = 2 * RP + SP + 64;
  static constexpr int DWORDS = 2 * RP + 2 * SP + 64;
  static constexpr int WAVES = 4;
  static constexpr int BYTES = WAVES * DWORDS * 4;
};

template <class S>
__device__ __forceinline__ CQ35_LDS uint32_t* down_stage(const Mega& m, int fw) {
  return (CQ35_LDS uint32_t*)(m.big + (size_t)fw * DownLayout<S>::DWORDS * 4);
}

// DMA one BF16 row of `elems` (a multiple of 8) into LDS at dst.
__device__ __forceinline__ void dma_row(const Mega& m, const uint16_t* src, CQ35_LDS uint32_t* dst, int elems) {
  const int pieces = elems / 8;  // 16-byte pieces
  for (int c = 0; c * 64 < pieces; ++c)
    if (m.lane + 64 * c < pieces)
      __builtin_amdgcn_global_load_lds(
          (const CQ35_GLOBAL void*)(src + (size_t)(m.lane + 64 * c) * 8), (CQ35_LDS void*)(dst + 256 * c), 16, 0, 0);
}

template <class S>
__device__ __forceinline__ void issue_down(const Mega& m, const CQ35_CONST MegaLayer& Ly) {
  using D = DownLayout<S>;
  const int fw = m.wave;
  const int prow = m.bid + m.grid * fw;
  if (fw >= D::WAVES || prow >= S::H / 2) return;
  CQ35_LDS uint32_t* st = down_stage<S>(m, fw);
#pragma unroll 1
  for (int slot = 0; slot < S::K; ++slot) {
    const int id = __builtin_amdgcn_readfirstlane(m.misc->ids[slot]);
    const uint16_t* w = Ly.down_exps + ((size_t)id * S::H + 2 * prow) * S::I;
    dma_row(m, w, st + D::A_R + slot * D::IP, S::I);
    dma_row(m, w + S::I, st + D::B_R + slot * D::IP, S::I);
  }
  const uint16_t* sw = Ly.sdown + (size_t)(2 * prow) * S::SI;
  dma_row(m, sw, st + D::A_S, S::SI);
  dma_row(m, sw + S::SI, st + D::B_S, S::SI);
}

// Dual S256 gate/up rows of the selected experts (moe.hex:254-333):
// bf16(silu(g) * u * p_slot), one row pair per wave.
template <class S>
__device__ __forceinline__ void phase_gate_up(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int l) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  constexpr int H = S::H, QH = S::QH, NQ = S::NQA;
  constexpr int PAIRS = S::K * S::I / 2;
  u32x4 gv[2][NQ], uv[2][NQ];
  poll_words<(S::E + 1 + kMT - 1) / kMT>(m, S::E + 1, Span{Ly.x_router},
                                          reinterpret_cast<uint32_t*>(m.misc->logits));
  select_experts<S>(m);
  trace_mark(kMarkSelected);
  // every block ranks the same logits; block 0 reports the layer's choice
  if (m.bid == 0 && m.tid < S::K) G(m.a.ids_out)[l * S::K + m.tid] = m.misc->ids[m.tid];
  const int p = m.gw;
  const bool has_pair = p < PAIRS;
  if (has_pair) {
    // both rows of a pair lie in one expert slot (I is even)
    const int slot = (2 * p) / S::I;
    const int id = __builtin_amdgcn_readfirstlane(m.misc->ids[slot]);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const size_t e = (size_t)id * S::I + (2 * p + r - slot * S::I);
      const uint16_t* g = Ly.gate_exps + e * H;
      const uint16_t* u = Ly.up_exps + e * H;
#pragma unroll
      for (int j = 0; j < NQ; ++j) {
        const uint32_t off = (uint32_t)min(m.lane + 64 * j, QH - 1) * 16u;
        gv[r][j] = ldq_at(g, off);
        uv[r][j] = ldq_at(u, off);
      }
    }
  }
  if (has_pair) {
    uint16_t y[2];
    float xl[NQ][4], xh[NQ][4];
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      const u32x4 xq = (QH % 64 == 0 || m.lane + 64 * j < QH) ? m.xn[m.lane + 64 * j] : u32x4{0u, 0u, 0u, 0u};
      quad_unpack(xq, xl[j], xh[j]);
    }
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      Quad ga, ua;
      quad_zero(ga);
      quad_zero(ua);
#pragma unroll
      for (int j = 0; j < NQ; ++j)
        if (QH % 64 == 0 || m.lane + 64 * j < QH) {
          quad_acc_f(ga, xl[j], xh[j], gv[r][j]);
          quad_acc_f(ua, xl[j], xh[j], uv[r][j]);
        }
      const float t = quad_tree64_pair_end(ga, ua);  // gate total in lane 31, up total in lane 63
      const float gb = rbf(lane_value(t, 31)), ub = rbf(lane_value(t, 63));
      y[r] = f2bf((silu(gb) * ub) * m.misc->probs[(2 * p + r) / S::I]);
    }
    if (m.lane == 0) word_store(Ly.x_active + p, pack_bf(y[0], y[1]), m.tag);
  }
  trace_mark(kMarkGateUpDone);
  // the down-projection rows of the selected experts, once this wave's
  // outputs are out (issued earlier, they hold the compute above behind the
  // memory queue); they land during the exchange into the down phase
  issue_down<S>(m, Ly);
}

// ------------------------------------------ phase: MoE down + residual (S32)

// Per hidden row (moe.hex:371-434, simt_moe.hex:36-287): S32 over the
// concatenated routed activations (pair p reads expert ids[p / (I/2)]) and a
// separate S32 over the shared activations, one reference lane per physical
// lane (lanes 0-31 row A, lanes 32-63 row B) reading the staged weights;
// out = bf16(bf16(routed + residual) (+) bf16(shared)). The shared
// activations are completed here: bf16(t * sigmoid(shared logit)). Once its
// outputs are stored, the block issues the next layer's first projection
// weights.
template <class S>
__device__ __forceinline__ void phase_down(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly,
                                           const MegaLayer* next, ProjRegs<S>& pr) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  using D = DownLayout<S>;
  constexpr int H = S::H, RP = D::RP, SP = D::SP;
  constexpr int NJ = RP / 32, NSJ = SP / 32;
  const uint64_t* act = Ly.x_active;
  const uint64_t* shr = Ly.x_shared;
  const uint64_t* lge = Ly.x_router + S::E;
  poll_words<(RP + SP + 1 + kMT - 1) / kMT>(
      m, RP + SP + 1, [&](int i) { return i < RP ? act + i : i < RP + SP ? shr + (i - RP) : lge; }, m.vec);
  // the staged weights were issued before the poll: complete in issue order
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if (m.tid < SP) {
    const float gate = sigmoid(bitsf(m.vec[RP + SP]));
    const uint32_t t = m.vec[RP + m.tid];
    m.vec[RP + m.tid] = pack_bf(f2bf(lo2f(t) * gate), f2bf(hi2f(t) * gate));
  }
  __syncthreads();
  trace_mark(kMarkDownStaged);
  const int half = m.lane >> 5, r32 = m.lane & 31;
  const int fw = m.wave;
  const int prow = m.bid + m.grid * fw;
  if (fw < D::WAVES && prow < H / 2) {
    const CQ35_LDS uint32_t* st = down_stage<S>(m, fw);
    const CQ35_LDS uint32_t* wr = st + (half ? D::B_R : D::A_R) + r32;
    const CQ35_LDS uint32_t* ws = st + (half ? D::B_S : D::A_S) + r32;
    float lo = 0.0f, hi = 0.0f;
    pair_chain_lds<NJ>(lo, hi, m.vec + r32, wr);
    const float routed_v = tree32_lanes(lo + hi);
    float slo = 0.0f, shi = 0.0f;
    pair_chain_lds<NSJ>(slo, shi, m.vec + RP + r32, ws);
    const float shared_v = tree32_lanes(slo + shi);
    const int row = 2 * prow + half;
    const uint16_t out = bf_add(f2bf(routed_v + bf2f(m.xa[row])), f2bf(shared_v));
    const uint16_t other = (uint16_t)__shfl_down((int)out, 32, 64);
    if (m.lane == 0) word_store(Ly.x_out + prow, pack_bf(out, other), m.tag);
  }
  trace_mark(kMarkDownDone);
  // the next layer's first projection pairs, once this block's outputs are
  // out (issuing them earlier stalls the compute above behind the memory
  // queue): they stream during the next exchange
  if (next) {
    issue_project<S, 0, kPairsEarly>(pa, next, pr);
  } else {
    // defined on every path, so the registers are not carried across phases
#pragma unroll
    for (int k = 0; k < kPairsEarly; ++k)
#pragma unroll
      for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int j = 0; j < S::NQA; ++j) pr.w[k][rr][j] = u32x4{0u, 0u, 0u, 0u};
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
// of that position into the cache for later steps.
struct ScoreLds {
  float rope[256];
  float normed[kMW][256];
  float qhat[16 * 256];  // normalised query heads, lane-major (channel l32 + 32 j at l32 * KJ + j)
  uint16_t khat[2 * 256];
  int heads[32];  // heads this block normalises: query heads, then Q + key head
  int nheads;
};
static_assert(sizeof(ScoreLds) <= kLdsBigBytes, "score LDS");
static_assert(offsetof(ScoreLds, qhat) % 16 == 0, "16-byte reads of the query heads");

// Head RMS norm with the adjacent-pair tree and neox RoPE on the first R
// channels (full_prepare.hex:3-82) of the heads listed in s->heads, one wave
// per head: a head index hh < Q is query head hh, Q + g key head g. src(hh)
// is the head's raw BF16 row; query heads land as F32 of their BF16 results
// in s->qhat, lane-major (channel l32 + 32 j of slot qslot(hh) at
// (qslot * HD) + l32 * KJ + j), key heads as BF16 in s->khat[g * HD + c].
// Needs s->rope filled and a barrier before.
template <class S, class L, class Src, class QSlot>
__device__ __forceinline__ void prepare_heads(const Mega& m, L* s, int nheads, const float (&qw_)[S::HD / 64],
                                              const float (&kw_)[S::HD / 64], Src src, QSlot qslot) {
  constexpr int HD = S::HD, Q = S::Q, KVH = S::KVH, KJ = HD / 32, RH = S::R / 2, VPL = HD / 64;
  const CQ35_CONST MegaArgs& a = m.a;
#pragma unroll 1
  for (int h0 = 0; h0 < nheads; h0 += kMW) {
    const bool live = h0 + m.wave < nheads;
    const int hh = live ? s->heads[h0 + m.wave] : Q + KVH;
    const bool is_q = hh < Q;
    float x[VPL], w[VPL];
    float t = 0.0f;
    if (hh < Q + KVH) {
      const uint16_t* row = src(hh);
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        x[i] = bf2f(row[VPL * m.lane + i]);
        w[i] = is_q ? qw_[i] : kw_[i];
      }
      // adjacent-pair tree: in-lane pairs first, then the lanes
      if constexpr (VPL == 1) t = x[0] * x[0];
      else if constexpr (VPL == 2) t = x[0] * x[0] + x[1] * x[1];
      else t = (x[0] * x[0] + x[1] * x[1]) + (x[2] * x[2] + x[3] * x[3]);
    }
    t = t + lane_down<1>(t);
    t = t + lane_down<2>(t);
    t = t + lane_down<4>(t);
    t = t + lane_down<8>(t);
    t = t + lane_down<16>(t);
    t = t + lane_down<32>(t);
    const float sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, t)));
    if (hh < Q + KVH) {
      const float inverse = 1.0f / nsqrt(sum / (float)HD + a.eps);
#pragma unroll
      for (int i = 0; i < VPL; ++i)
        s->normed[m.wave][VPL * m.lane + i] = bf2f(bf_mul(f2bf(x[i] * inverse), f2bf(w[i])));
    }
    __syncthreads();
    if (hh < Q + KVH) {
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = m.lane + 64 * i;
        const float nf = s->normed[m.wave][c];
        float result = nf;
        if (c < S::R) {
          const int pair = c % RH;
          const bool first = c < RH;
          const float partner = s->normed[m.wave][first ? pair + RH : pair];
          const float ac = nf * s->rope[pair];
          const float bs = partner * s->rope[pair + RH];
          result = first ? ac - bs : ac + bs;
        }
        const uint16_t rb = f2bf(result);
        if (is_q) s->qhat[qslot(hh) * HD + (c & 31) * KJ + (c >> 5)] = bf2f(rb);
        else s->khat[(hh - Q) * HD + c] = rb;
      }
    }
    __syncthreads();
  }
}

template <class S>
__device__ __forceinline__ void phase_scores(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, Q = S::Q, KVH = S::KVH, HPK = Q / KVH, KJ = HD / 32, RH = S::R / 2;
  static_assert(Q * HD <= 16 * 256 && KVH * HD <= 2 * 256 && KJ % 2 == 0, "score shape");
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int64_t items = keys * KVH;
  ScoreLds* s = reinterpret_cast<ScoreLds*>(m.big);
  const int l32 = m.lane & 31, half = m.lane >> 5;
  // the block's items are 16 consecutive ones per round; without any it has
  // nothing to do in this phase
  const int64_t first = (int64_t)m.bid * 2 * kMW;
  if (first >= items) return;  // uniform per block
  // item indices fit 32 bits (capacity <= 2^18, KVH <= 8): 32-bit division
  const uint32_t ukeys = (uint32_t)keys, uitems = (uint32_t)items;
  // score items: two per wave (32 lanes each) per round, in batches of SB
  // rounds whose cached keys are read one batch ahead (reads of invalid
  // rounds are clamped to key 0 and ignored); the first batch is read now
  constexpr int SB = 4;
  const int64_t item0 = (int64_t)m.gw * 2 + half;
  const int64_t stride = 2 * (int64_t)m.nw;
  const int rounds = item0 < items ? (int)((items - 1 - item0) / stride) + 1 : 0;
  const int nb = (rounds + SB - 1) / SB;
  auto load_batch = [&](uint32_t (&kv)[SB][KJ], int b) {
#pragma unroll
    for (int rr = 0; rr < SB; ++rr) {
      const uint32_t it = (uint32_t)(item0 + (int64_t)(b * SB + rr) * stride);
      uint32_t kvh = 0, key = 0;
      if (it < uitems) {
        kvh = it / ukeys;
        key = it - kvh * ukeys;
        if (key >= (uint32_t)position) key = 0;
      }
      const uint16_t* kr = a.cache + Ly.key_base + (int64_t)key * S::KVS + (int64_t)kvh * HD + l32;
#pragma unroll
      for (int j = 0; j < KJ; ++j) kv[rr][j] = G(kr)[32 * j];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the batch being scored
  };
  uint32_t ka[SB][KJ], kb[SB][KJ];
  if (nb > 0) load_batch(ka, 0);
  // norm weights (shared by all query heads / all key heads) and the RoPE
  // frequencies do not depend on the projection: load them first
  constexpr int VPL = HD / 64;  // values per lane
  float qw_[VPL], kw_[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    qw_[i] = G(Ly.qnorm)[VPL * m.lane + i];
    kw_[i] = G(Ly.knorm)[VPL * m.lane + i];
  }
  const float freq = G(a.freq)[min(m.tid, RH - 1)];
  // query parts of every head, then the raw key and value heads
  constexpr int QWORDS = Q * (HD / 2), KVWORDS = S::KVS / 2;
  auto index = [&](int i) -> int {
    if (i < QWORDS) {
      const int hq = i / (HD / 2), c = i - hq * (HD / 2);
      return hq * HD + c;  // words of [q(HD) | gate(HD)] per head
    }
    return S::QS + (i - QWORDS);  // k words then v words
  };
  const uint64_t* proj = Ly.x_proj;
  poll_words<(QWORDS + 2 * KVWORDS + kMT - 1) / kMT>(m, QWORDS + 2 * KVWORDS,
                                                     [&](int i) { return proj + index(i); }, m.vec);
  const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
  const uint16_t* kraw = in16 + Q * HD;
  const uint16_t* vraw = kraw + S::KVS;
  // KV groups touched by the block's items -> heads to normalise
  if (m.tid == 0) {
    // windows of 2 kMW items start every 2 nw items from `first`; when a KV
    // group holds at least that many items, no group between the first and
    // the last window's is skipped
    const uint32_t ustride = 2u * (uint32_t)m.nw, ufirst = (uint32_t)first;
    const uint32_t ulast_start = ufirst + (uitems - 1 - ufirst) / ustride * ustride;
    unsigned mask = 0;
    if (ukeys >= ustride) {
      const uint32_t g0 = ufirst / ukeys, g1 = min(ulast_start + 2u * kMW, uitems) - 1u;
      for (uint32_t g = g0; g <= g1 / ukeys; ++g) mask |= 1u << g;
    } else {
      for (uint32_t i0 = ufirst; i0 < uitems; i0 += ustride) {
        const uint32_t i1 = min(i0 + 2u * kMW, uitems) - 1u;
        for (uint32_t g = i0 / ukeys; g <= i1 / ukeys; ++g) mask |= 1u << g;
      }
    }
    int n = 0;
    for (int g = 0; g < KVH; ++g)
      if (mask & (1u << g)) {
        for (int hq = 0; hq < HPK; ++hq) s->heads[n++] = g * HPK + hq;
        s->heads[n++] = Q + g;
      }
    s->nheads = n;
  }
  // RoPE table for this position (rope.hex:5-17)
  if (m.tid < RH) {
    float sn, cs;
    sincos_q((float)(uint32_t)position * freq, &sn, &cs);
    s->rope[m.tid] = cs;
    s->rope[RH + m.tid] = sn;
  }
  __syncthreads();
  // one wave per head of the list
  prepare_heads<S>(m, s, s->nheads, qw_, kw_, [&](int hh) {
    return hh < Q ? in16 + hh * HD : kraw + (hh - Q) * HD;
  }, [&](int hh) { return hh; });
  auto score_batch = [&](const uint32_t (&kv)[SB][KJ], int b) {
#pragma unroll
    for (int rr = 0; rr < SB; ++rr) {
      const uint32_t it = (uint32_t)(item0 + (int64_t)(b * SB + rr) * stride);
      if (it >= uitems) continue;
      const int kvh = (int)(it / ukeys);
      const int64_t key = (int64_t)(it - (uint32_t)kvh * ukeys);
      float kf[KJ];
      if (key == position) {
#pragma unroll
        for (int j = 0; j < KJ; ++j) kf[j] = bf2f(s->khat[kvh * HD + l32 + 32 * j]);
        // K and V of the new position into the cache, for later steps (this
        // step's values phase takes V from the projection words)
        uint16_t* kdst = a.cache + Ly.key_base + position * S::KVS + (int64_t)kvh * HD;
        uint16_t* vdst = a.cache + Ly.value_base + position * S::KVS + (int64_t)kvh * HD;
#pragma unroll
        for (int j = 0; j < KJ; ++j) {
          const int c = l32 + 32 * j;
          G(kdst)[c] = s->khat[kvh * HD + c];
          G(vdst)[c] = vraw[kvh * HD + c];
        }
      } else {
#pragma unroll
        for (int j = 0; j < KJ; ++j) kf[j] = bf2f((uint16_t)kv[rr][j]);
      }
#pragma unroll
      for (int hq = 0; hq < HPK; ++hq) {
        const int head = kvh * HPK + hq;
        const float* qh = s->qhat + head * HD + l32 * KJ;
        float qv[KJ];
        if constexpr (KJ % 4 == 0) {
#pragma unroll
          for (int w = 0; w < KJ / 4; ++w) {
            const f32x4 t = reinterpret_cast<const f32x4*>(qh)[w];
            qv[4 * w] = t.x; qv[4 * w + 1] = t.y; qv[4 * w + 2] = t.z; qv[4 * w + 3] = t.w;
          }
        } else {
#pragma unroll
          for (int j = 0; j < KJ; ++j) qv[j] = qh[j];
        }
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < KJ; ++j) acc += qv[j] * kf[j];
        acc = tree32_lanes(acc);  // halving strides 16 .. 1 in each half wave
        if (l32 == 0) word_store(Ly.x_scores + (size_t)head * a.cap + key, fbits(acc * a.attn_scale), m.tag);
      }
    }
  };
  int b = 0;
#pragma unroll 1
  for (; b + 1 < nb; b += 2) {
    load_batch(kb, b + 1);
    score_batch(ka, b);
    load_batch(ka, min(b + 2, nb - 1));
    score_batch(kb, b + 1);
  }
  if (b < nb) score_batch(ka, b);
  __syncthreads();
}

// ------------------------------------- phase: attention values (full layers)

// Per (query head, 16-channel chunk) item, the reference's online softmax in
// 8-key tiles (online.hex:272-331; per-kernel version attention.h). Every
// channel's accumulator is one serial chain acc = acc * alpha_t + prod_0 +
// ... + prod_7 over the tiles (contraction off), so the phase is bound by
// that chain's dependent-op latency. A three-stage pipeline over chunks of
// kMegaValueChunk keys keeps everything else off it, one barrier a chunk:
//  - scan (wave 2), chunk i: polls the chunk's score words (fetched two
//    chunks ahead), keeps the scores in LDS, takes the tile maxima and their
//    running maximum (a prefix maximum across the wave carried from the
//    previous chunk: max is exact, so any association gives the reference's
//    values) and alpha_t = exp(m_{t-1} - m_t);
//  - products (waves 4-7), chunk i-1: p_k = exp(s_k - m_t) and every product
//    p_k * v_{k,c} (each rounds on its own in the reference too), V rows
//    fetched three chunks ahead;
//  - chains, chunk i-2: wave 0 runs the 16 channel chains, wave 1 the
//    denominator chain den = den * alpha_t + p_0 + ... + p_7. A chunk whose
//    alphas are all exactly 1 skips the multiplications (x * 1 == x).
// out = bf16(bf16(acc / den) * sigmoid(gate)). Invalid keys of the last tile
// contribute p = 0 against key 0's value, as in the reference. The new
// position's V comes from the projection words (the cache copy is written by
// the scores phase for later steps).
constexpr int kMegaValueChunk = 256;              // keys per chunk
constexpr int kValueTiles = kMegaValueChunk / 8;  // tiles per chunk
constexpr int kProdStride = kMegaValueChunk + 4;  // padded channel rows of the products
constexpr int kValueRing = 3;                     // chunks of V rows in flight per producer
constexpr int kScoreRing = 3;                     // chunks of score words in flight on the scan wave
static_assert(kValueRing == 3 && kScoreRing == 3, "the role loops unroll by the ring depth");
struct ValueLds {
  float prod[2][kValueChannels * kProdStride];  // [buffer][channel][key]
  float p[2][kMegaValueChunk];
  float sc[3][kMegaValueChunk];
  float alpha[3][kValueTiles];
  float mx[3][kValueTiles];
  int one[3];
  uint32_t vnew[kValueChannels / 2];
  float den[4];
};
static_assert(sizeof(ValueLds) <= kLdsBigBytes, "value LDS");
static_assert(kProdStride % 4 == 0 && offsetof(ValueLds, p) % 16 == 0 && offsetof(ValueLds, sc) % 16 == 0 &&
                  offsetof(ValueLds, alpha) % 16 == 0 && sizeof(ValueLds::alpha[0]) % 16 == 0,
              "16-byte reads of the value stages");
static_assert(kMegaValueChunk == 4 * 64 && kMegaValueChunk == 2 * 128, "lane mapping of the value stages");

// One channel chain (or the denominator chain) over the tiles t = s, s + ns,
// ... below nt of a chunk: row holds the tiles' eight addends in key order,
// alpha the tiles' rescale factors. Four tiles make a group; two register
// sets alternate, so the next group's addends are read while the current
// group is summed, with no copies on the chain's wave (the last read is
// clamped to a valid group). With ns = 1 this is every tile in order.
template <bool SCALE>
__device__ __forceinline__ float chain_group(float acc, const f32x4 (&x)[8], const float (&al)[4]) {
#pragma unroll
  for (int t = 0; t < 4; ++t) {
    if (SCALE) acc = acc * al[t];
    const f32x4 x0 = x[2 * t], x1 = x[2 * t + 1];
    acc = acc + x0.x; acc = acc + x0.y; acc = acc + x0.z; acc = acc + x0.w;
    acc = acc + x1.x; acc = acc + x1.y; acc = acc + x1.z; acc = acc + x1.w;
  }
  return acc;
}

template <bool SCALE>
__device__ __forceinline__ float value_chain(float acc, const f32x4* row, const float* alpha, int nt, int s,
                                             int ns) {
  const int count = s < nt ? (nt - 1 - s) / ns + 1 : 0;  // this split's tiles in the chunk
  const int groups = count >> 2;
  f32x4 xa[8], xb[8];
  float aa[4], ab[4];
  // the scheduler would sink the reads next to their first use; the
  // barrier keeps them issued ahead of the group being summed
  auto load = [&](f32x4 (&x)[8], float (&al)[4], int g) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = s + ns * (4 * g + u);
      x[2 * u] = row[2 * t];
      x[2 * u + 1] = row[2 * t + 1];
      if (SCALE) al[u] = alpha[t];
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  if (groups > 0) load(xa, aa, 0);
  int g = 0;
#pragma unroll 1
  for (; g + 1 < groups; g += 2) {
    load(xb, ab, g + 1);
    acc = chain_group<SCALE>(acc, xa, aa);
    load(xa, aa, min(g + 2, groups - 1));
    acc = chain_group<SCALE>(acc, xb, ab);
  }
  if (g < groups) acc = chain_group<SCALE>(acc, xa, aa);
#pragma unroll 1
  for (int j = 4 * groups; j < count; ++j) {
    const int t = s + ns * j;
    if (SCALE) acc = acc * alpha[t];
    const f32x4 x0 = row[2 * t], x1 = row[2 * t + 1];
    acc = acc + x0.x; acc = acc + x0.y; acc = acc + x0.z; acc = acc + x0.w;
    acc = acc + x1.x; acc = acc + x1.y; acc = acc + x1.z; acc = acc + x1.w;
  }
  return acc;
}

// XCD-aware item order. Workgroups are dispatched to the 8 XCDs round-robin
// (block b on XCD b % 8), each XCD with its own L2. For the 35B shape
// (2 KV heads x 8 query heads x 16 chunks of 16 channels = 256 items) XCD x
// takes KV head x / 4 and its chunks 4 (x % 4) .. +3 for all 8 query heads:
// the 128-byte V segment of every key row is fetched from HBM by one XCD and
// reused from its L2 by the query heads, instead of each line being fetched
// by the four XCDs that read its 32-byte chunks. Other shapes keep the
// natural order. A bijection on [0, ITEMS): only the placement changes.
template <class S>
__device__ __forceinline__ int value_item(int slot) {
  constexpr int HPK = S::Q / S::KVH, CHUNKS = S::HD / kValueChannels;
  if constexpr (S::KVH == 2 && HPK == 8 && CHUNKS == 16) {
    const int x = slot & 7, s = slot >> 3;
    return ((x >> 2) * HPK + (s >> 2)) * CHUNKS + 4 * (x & 3) + (s & 3);
  } else {
    return slot;
  }
}

template <class S>
__device__ __forceinline__ void phase_values(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int tb) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, HPK = S::Q / S::KVH, CHUNKS = HD / kValueChannels, ITEMS = S::Q * CHUNKS;
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int tiles = (int)((keys + 7) >> 3);
  const int64_t padded = (int64_t)tiles * 8;
  const int nch = (int)((padded + kMegaValueChunk - 1) / kMegaValueChunk);
  ValueLds* s = reinterpret_cast<ValueLds*>(m.big);
  const float ninf = bitsf(0xff800000u);
  // one chain over every tile (split-K contexts take phase_flash instead)
  constexpr int ns = 1;
  constexpr int sp = 0;
  const int pj = m.tid - 4 * 64;  // producer thread (waves 4-7)
  const int ph = pj & 1;          // channels 8 ph .. 8 ph + 7
#pragma unroll 1
  for (int slot = m.bid; slot < ITEMS; slot += m.grid) {
    const int item = value_item<S>(slot);
    const int head = item / CHUNKS, c0 = (item - head * CHUNKS) * kValueChannels;
    const uint16_t* vbase = a.cache + Ly.value_base + (int64_t)(head / HPK) * HD + c0 + 8 * ph;
    const uint64_t* sc = Ly.x_scores + (size_t)head * a.cap;
    // V quad of key k (key 0 past the end); nothing past the last tile
    auto load_v = [&](int64_t k) -> u32x4 {
      if (k >= padded) return u32x4{0u, 0u, 0u, 0u};
      const int64_t safe = k < keys ? k : 0;
      return G(reinterpret_cast<const u32x4*>(vbase + safe * S::KVS))[0];
    };
    // score word of key k (a ready placeholder past the last key)
    auto load_s = [&](int64_t k) -> uint64_t {
      return k < keys ? word_load(sc + k) : ((uint64_t)m.tag << 32);
    };
    // Each role runs its own loop of n_iter iterations with one barrier each
    // (every wave passes the same barriers); the prefetch rings are indexed
    // by chunk mod 3 through unrolling, so a ring slot is only waited on
    // three chunks after its reads were issued.
    const int n_iter = nch + 2;
    using R0 = std::integral_constant<int, 0>;
    using R1 = std::integral_constant<int, 1>;
    using R2 = std::integral_constant<int, 2>;
    uint32_t gate_word = 0;
    float acc = 0.0f, den = 0.0f;
    RoleClock clk;  // phase-trace builds: this role's busy time
    clk.resume();
    if (m.wave <= 1) {
      if (m.wave == 0) {
        if (m.lane < kValueChannels / 2)
          gate_word = poll_one(m, Ly.x_proj + ((head * 2 * HD + HD + c0) >> 1) + m.lane);
      } else if (m.lane < kValueChannels / 2) {
        // the new position's V (word pairs of the projection)
        s->vnew[m.lane] = poll_one(m, Ly.x_proj + (S::QS + S::KVS / 2 + ((head / HPK * HD + c0) >> 1)) + m.lane);
      }
#pragma unroll 1
      for (int i = 0; i < n_iter; ++i) {
        const int c = i - 2;
        if (c >= 0) {
          const int slot = c % 3, buf = c & 1;
          const int nt = min(kValueTiles, tiles - c * kValueTiles);
          const bool one = s->one[slot] != 0;
          if (m.wave == 0) {
            const f32x4* row = reinterpret_cast<const f32x4*>(s->prod[buf] + (m.lane & 15) * kProdStride);
            acc = one ? value_chain<false>(acc, row, s->alpha[slot], nt, sp, ns)
                      : value_chain<true>(acc, row, s->alpha[slot], nt, sp, ns);
          } else {
            const f32x4* row = reinterpret_cast<const f32x4*>(s->p[buf]);
            den = one ? value_chain<false>(den, row, s->alpha[slot], nt, sp, ns)
                      : value_chain<true>(den, row, s->alpha[slot], nt, sp, ns);
            if ((m.lane & 15) == 0) s->den[sp] = den;
          }
        }
        clk.pause();
        __syncthreads();
        clk.resume();
      }
    } else if (m.wave == 2) {
      uint64_t sr[kScoreRing][4];  // slot r: chunks = r mod 3
#pragma unroll
      for (int r = 0; r < kScoreRing; ++r)
#pragma unroll
        for (int j = 0; j < 4; ++j) sr[r][j] = load_s((int64_t)r * kMegaValueChunk + 4 * m.lane + j);
      float carry = ninf;
      auto scan = [&](auto rr, int i) {
        constexpr int r = decltype(rr)::value;
        if (i < nch) {
          const int slot = i % 3;
          const int64_t k0 = (int64_t)i * kMegaValueChunk;
          uint64_t v[4];
#pragma unroll
          for (int j = 0; j < 4; ++j) v[j] = sr[r][j];
          unsigned spins = 0;
          while (true) {
            bool ready = true;
#pragma unroll
            for (int j = 0; j < 4; ++j) ready &= word_ready(v[j], m.tag);
            if (ready || spin_stop(m, ++spins)) break;
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (!word_ready(v[j], m.tag)) v[j] = load_s(k0 + 4 * m.lane + j);
          }
#pragma unroll
          for (int j = 0; j < 4; ++j)
            sr[r][j] = load_s(k0 + (int64_t)kScoreRing * kMegaValueChunk + 4 * m.lane + j);
          f32x4 sv;
          sv.x = bitsf((uint32_t)v[0]); sv.y = bitsf((uint32_t)v[1]);
          sv.z = bitsf((uint32_t)v[2]); sv.w = bitsf((uint32_t)v[3]);
          reinterpret_cast<f32x4*>(s->sc[slot])[m.lane] = sv;
          const int64_t kl = k0 + 4 * m.lane;
          float mt = fmaxf(fmaxf(kl < keys ? sv.x : ninf, kl + 1 < keys ? sv.y : ninf),
                           fmaxf(kl + 2 < keys ? sv.z : ninf, kl + 3 < keys ? sv.w : ninf));
          mt = fmaxf(mt, __shfl_xor(mt, 1, 64));  // the tile's two lanes
          // running maximum over the split's tiles (lanes 2 ns apart): a
          // prefix maximum is exact in any association
          float run = mt;
          for (int d = 2 * ns; d < 64; d <<= 1) {
            const float o = __shfl_up(run, d, 64);
            if (m.lane >= d) run = fmaxf(run, o);
          }
          run = fmaxf(run, carry);
          float prev = __shfl_up(run, 2 * ns, 64);
          if (m.lane < 2 * ns) prev = i == 0 ? ninf : carry;
          const float al = hexp(prev - run);
          const int t = m.lane >> 1;
          const bool valid = (m.lane & 1) == 0 && (int64_t)i * kValueTiles + t < tiles;
          if (valid) {
            s->mx[slot][t] = run;
            s->alpha[slot][t] = al;
          }
          const uint64_t scaled = __ballot(valid && al != 1.0f);
          if (m.lane == 0) s->one[slot] = scaled == 0ull ? 1 : 0;
          carry = __shfl(run, 64 - 2 * ns + 2 * ((m.lane >> 1) & (ns - 1)), 64);
        }
        clk.pause();
        __syncthreads();
        clk.resume();
      };
      int i = 0;
#pragma unroll 1
      for (; i + 3 <= n_iter; i += 3) {
        scan(R0{}, i);
        scan(R1{}, i + 1);
        scan(R2{}, i + 2);
      }
      if (i < n_iter) scan(R0{}, i);
      if (i + 1 < n_iter) scan(R1{}, i + 1);
    } else if (m.wave >= 4) {
      u32x4 vr[kValueRing][2];  // slot r: chunks = r mod 3
#pragma unroll
      for (int r = 0; r < kValueRing; ++r)
#pragma unroll
        for (int q = 0; q < 2; ++q)
          vr[r][q] = load_v((int64_t)r * kMegaValueChunk + (pj >> 1) + 128 * q);
      auto produce = [&](auto rr, int i) {
        constexpr int r = decltype(rr)::value;
        const int c = i - 1;
        if (c >= 0 && c < nch) {
          const int slot = c % 3, buf = c & 1;
          const int64_t k0 = (int64_t)c * kMegaValueChunk;
          u32x4 vnew;
          {
            const uint32_t* w = s->vnew + 4 * ph;
            vnew = u32x4{w[0], w[1], w[2], w[3]};
          }
#pragma unroll
          for (int q = 0; q < 2; ++q) {
            const int kk = (pj >> 1) + 128 * q;
            const int64_t k = k0 + kk;
            if (k < padded) {
              const float pk = k < keys ? hexp(s->sc[slot][kk] - s->mx[slot][kk >> 3]) : 0.0f;
              const u32x4 vq = k == position ? vnew : vr[r][q];
              float* dst = s->prod[buf] + (8 * ph) * kProdStride + kk;
              dst[0 * kProdStride] = pk * lo2f(vq.x); dst[1 * kProdStride] = pk * hi2f(vq.x);
              dst[2 * kProdStride] = pk * lo2f(vq.y); dst[3 * kProdStride] = pk * hi2f(vq.y);
              dst[4 * kProdStride] = pk * lo2f(vq.z); dst[5 * kProdStride] = pk * hi2f(vq.z);
              dst[6 * kProdStride] = pk * lo2f(vq.w); dst[7 * kProdStride] = pk * hi2f(vq.w);
              if (ph == 0) s->p[buf][kk] = pk;
            }
          }
#pragma unroll
          for (int q = 0; q < 2; ++q)
            vr[r][q] = load_v(k0 + (int64_t)kValueRing * kMegaValueChunk + (pj >> 1) + 128 * q);
        }
        clk.pause();
        __syncthreads();
        clk.resume();
      };
      // iteration i produces chunk i - 1, whose ring slot is (i + 2) mod 3
      int i = 0;
#pragma unroll 1
      for (; i + 3 <= n_iter; i += 3) {
        produce(R2{}, i);
        produce(R0{}, i + 1);
        produce(R1{}, i + 2);
      }
      if (i < n_iter) produce(R2{}, i);
      if (i + 1 < n_iter) produce(R0{}, i + 1);
    } else {
#pragma unroll 1
      for (int i = 0; i < n_iter; ++i) __syncthreads();
    }
    // role busy times: scan (wave 2), products (waves 4-7, summed), channel
    // chains (wave 0), denominator chain (wave 1)
    if (m.wave <= 2 || m.wave >= 4)
      trace_add(tb + 14 + (m.wave == 2 ? 0 : m.wave >= 4 ? 1 : m.wave == 0 ? 2 : 3), clk.busy);
    if (m.wave == 0) {
      den = s->den[0];
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


// ------------------------- phases: split-K attention (long contexts only)

// Above the session's split threshold a full layer's attention runs as at
// most kSplitRanges ranges of ceil(T / kSplitRanges) 8-key tiles per KV head
// (T tiles in all): phase_flash gives every (KV head, range) item to a block,
// which prepares the group's query heads, scores the range's keys for all of
// them (each key row read once), runs the reference's online recurrence over
// the range's tiles from scratch (its running maximum, alphas, denominator
// and per-channel accumulators, the orders of phase_scores and
// phase_values) and publishes (m_r, den_r, acc_r[HD]) per query head as
// tagged words. phase_merge then folds the ranges in ascending order for each
// (query head, 16-channel) item: M = max_r m_r, w_r = exp(m_r - M),
// den = 0 + den_0 w_0 + den_1 w_1 + ..., acc likewise,
// out = bf16(bf16(acc / den) * sigmoid(gate)). The per-kernel path
// (attention.h) and the restatement split the same way.
//
// A range is processed in sub-chunks of at most kFlashSubTiles tiles
// (balanced, multiples of 4 tiles) carrying the running maximum,
// denominator and accumulators, so the chain is the range's one recurrence.
// Per sub-chunk: V rows of its first kFlashDepth passes are requested, the
// keys are scored (query heads held in registers), each head's wave scans
// the tile maxima, then the V passes of kFlashVKeys rows run with the next
// kFlashDepth - 1 passes in flight (16-byte loads into a register ring).
constexpr int kFlashSubTiles = 64;
constexpr int kFlashVKeys = 32;  // V rows staged per pass
constexpr int kFlashDepth = 4;   // V passes in flight

struct FlashLds {
  float rope[256];
  float qhat[8 * 256];      // the group's query heads, lane-major
  uint16_t khat[2 * 256];   // key heads (the new position's)
  uint16_t vnew[256];       // the new position's value head
  float alpha[8][kFlashSubTiles];
  float mr[8];              // each head's running maximum (carried over sub-chunks)
  int heads[32];
  int nheads;
  int pad[3];
  union {
    float normed[kMW][256];                 // prepare_heads only
    float p[8][8 * kFlashSubTiles];         // scores, then weights, per query head of the group
  };
  uint16_t v[kFlashVKeys][256];  // V rows of the current pass
};
static_assert(sizeof(FlashLds) <= kLdsBigBytes, "flash LDS");
static_assert(offsetof(FlashLds, qhat) % 16 == 0 && offsetof(FlashLds, v) % 16 == 0 &&
                  offsetof(FlashLds, p) % 16 == 0,
              "16-byte LDS rows");

// Words per (query head, range) partial: m, den, acc[HD].
template <class S>
constexpr int flash_words() { return 2 + S::HD; }

// Phase-trace builds: per-stage time of the flash phase (prepare, scores,
// scan, values), added per block into the layer's slots 14-17, items in 18.
struct FlashClock {
#ifdef CQ35_PHASE_TRACE
  uint64_t t = __builtin_amdgcn_s_memrealtime(), spent[4] = {0, 0, 0, 0};
  __device__ __forceinline__ void lap(int i) {
    const uint64_t n = __builtin_amdgcn_s_memrealtime();
    spent[i] += n - t;
    t = n;
  }
  __device__ __forceinline__ void flush(int tb, int items) {
    if (threadIdx.x == 0) {
      for (int i = 0; i < 4; ++i) trace_lds()[tb + 14 + i] += spent[i];
      trace_lds()[tb + 18] += (uint64_t)items;
    }
  }
#else
  __device__ __forceinline__ void lap(int) {}
  __device__ __forceinline__ void flush(int, int) {}
#endif
};

template <class S>
__device__ __forceinline__ void phase_flash(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int tb) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, Q = S::Q, KVH = S::KVH, HPK = Q / KVH, KJ = HD / 32, RH = S::R / 2;
  constexpr int VPL = HD / 64, FW = flash_words<S>();
  static_assert(HPK <= 8 && HD <= 256 && KVH <= 2, "flash shape");
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int tiles = (int)((keys + 7) >> 3);
  const int rtiles = (tiles + kSplitRanges - 1) / kSplitRanges;  // tiles per range
  const int nranges = (tiles + rtiles - 1) / rtiles;
  FlashLds* s = reinterpret_cast<FlashLds*>(m.big);
  const float ninf = bitsf(0xff800000u);
  const int l32 = m.lane & 31, half = m.lane >> 5;
  FlashClock clk;
  float qw_[VPL], kw_[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    qw_[i] = G(Ly.qnorm)[VPL * m.lane + i];
    kw_[i] = G(Ly.knorm)[VPL * m.lane + i];
  }
  const float freq = G(a.freq)[min(m.tid, RH - 1)];
  int nitems = 0;
#pragma unroll 1
  for (int item = m.bid; item < KVH * nranges; item += m.grid) {
    ++nitems;
    const int g = item % KVH, r = item / KVH;
    const int nt = min(rtiles, tiles - r * rtiles);  // tiles of the range
    const int64_t k0 = (int64_t)r * rtiles * 8;
    const int n = (int)min<int64_t>(8 * nt, keys - k0);  // keys of the range
    const bool has_new = r == nranges - 1;                // the range holding the new position
    // the group's query parts, its key and value heads (projection words)
    constexpr int QW = HPK * (HD / 2), KW = HD / 2;
    const uint64_t* proj = Ly.x_proj;
    auto index = [&](int i) -> int {
      if (i < QW) {
        const int hq = i / (HD / 2), c = i - hq * (HD / 2);
        return (g * HPK + hq) * HD + c;  // words of [q(HD) | gate(HD)] per head
      }
      if (i < QW + KW) return S::QS + g * (HD / 2) + (i - QW);               // key head g
      return S::QS + S::KVS / 2 + g * (HD / 2) + (i - QW - KW);              // value head g
    };
    poll_words<(QW + 2 * KW + kMT - 1) / kMT>(m, QW + 2 * KW, [&](int i) { return proj + index(i); }, m.vec);
    const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
    if (m.tid == 0) {
      int nh = 0;
      for (int hq = 0; hq < HPK; ++hq) s->heads[nh++] = g * HPK + hq;
      if (has_new) s->heads[nh++] = Q + g;
      s->nheads = nh;
    }
    if (m.tid < HPK) s->mr[m.tid] = ninf;
    if (m.tid < RH) {
      float sn, cs;
      sincos_q((float)(uint32_t)position * freq, &sn, &cs);
      s->rope[m.tid] = cs;
      s->rope[RH + m.tid] = sn;
    }
    if (has_new && m.tid < HD) s->vnew[m.tid] = in16[QW * 2 + HD + m.tid];
    __syncthreads();
    prepare_heads<S>(m, s, s->nheads, qw_, kw_, [&](int hh) {
      return hh < Q ? in16 + (hh - g * HPK) * HD : in16 + QW * 2;
    }, [&](int hh) { return hh - g * HPK; });
    // the new position's K and V into the cache for later steps
    if (has_new && m.tid < HD) {
      uint16_t* kdst = a.cache + Ly.key_base + position * S::KVS + (int64_t)g * HD;
      uint16_t* vdst = a.cache + Ly.value_base + position * S::KVS + (int64_t)g * HD;
      G(kdst)[m.tid] = s->khat[g * HD + m.tid];
      G(vdst)[m.tid] = s->vnew[m.tid];
    }
    clk.lap(0);
    // sub-chunks: nsub of st tiles (a multiple of 4; the last may be shorter)
    const int nsub = (nt + kFlashSubTiles - 1) / kFlashSubTiles;
    const int st = (((nt + nsub - 1) / nsub) + 3) & ~3;
    // channel chains: thread = channels 2 cp, 2 cp + 1 of query heads 2 hp,
    // 2 hp + 1 (one 4-byte V read serves both channels, each head's 8
    // weights of a tile are two 16-byte LDS reads); threads tid < HPK also
    // run head tid's denominator chain
    static_assert(HPK % 2 == 0 && (HPK / 2) * (HD / 2) <= kMT, "flash chains");
    const int cp = m.tid % (HD / 2), hp = m.tid / (HD / 2);
    const bool chains = hp < HPK / 2;
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};  // [head][channel]
    float den = 0.0f;
    constexpr int VQ = kFlashVKeys * HD / 8;     // 16-byte quads per pass
    constexpr int VPT = (VQ + kMT - 1) / kMT;    // per thread
    u32x4 ring[kFlashDepth][VPT];
#pragma unroll 1
    for (int sc = 0; sc < nsub; ++sc) {
      const int t0 = sc * st;                    // first tile of the sub-chunk (range-relative)
      const int snt = min(st, nt - t0);          // its tiles
      const int c0 = 8 * t0;                     // its first key (range-relative)
      const int sn = min(8 * snt, n - c0);       // its keys
      const int np = (snt + 3) / 4;              // its V passes
      // V rows of pass q into ring registers (rows past the range read key
      // 0's row; their weight is 0; the new position's row comes from LDS)
      auto fetch = [&](u32x4 (&dst)[VPT], int q) {
        if (q >= np) return;
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
          const int idx = m.tid + kMT * i;
          if (VQ % kMT == 0 || idx < VQ) {
            const int kk = c0 + kFlashVKeys * q + idx / (HD / 8), qd = idx % (HD / 8);
            const int64_t key = kk < n ? k0 + kk : 0;
            if (key == position) dst[i] = reinterpret_cast<const u32x4*>(s->vnew)[qd];
            else dst[i] = G(reinterpret_cast<const u32x4*>(a.cache + Ly.value_base + key * S::KVS + (int64_t)g * HD))[qd];
          }
        }
      };
      auto put = [&](const u32x4 (&src)[VPT]) {
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
          const int idx = m.tid + kMT * i;
          if (VQ % kMT == 0 || idx < VQ) reinterpret_cast<u32x4*>(&s->v[idx / (HD / 8)][0])[idx % (HD / 8)] = src[i];
        }
      };
#pragma unroll
      for (int d = 0; d < kFlashDepth; ++d) fetch(ring[d], d);
      // scores: half-wave hw takes keys hw, hw + 16, ... of the sub-chunk;
      // lane l32 owns channels l32 + 32 j (serial from 0.0, then the 32-lane tree)
      const int hw = 2 * m.wave + half;
      constexpr int SB = 2;
      auto load_keys = [&](uint32_t (&kv)[SB][KJ], int b) {
#pragma unroll
        for (int rr = 0; rr < SB; ++rr) {
          const int kk = c0 + min(hw + 16 * (b * SB + rr), sn - 1);
          const int64_t key = k0 + kk == position ? 0 : k0 + kk;
          const uint16_t* kr = a.cache + Ly.key_base + key * S::KVS + (int64_t)g * HD + l32;
#pragma unroll
          for (int j = 0; j < KJ; ++j) kv[rr][j] = G(kr)[32 * j];
        }
        __builtin_amdgcn_sched_barrier(0);
      };
      auto score_keys = [&](const uint32_t (&kv)[SB][KJ], int b) {
        float kf[SB][KJ];
#pragma unroll
        for (int rr = 0; rr < SB; ++rr) {
#pragma unroll
          for (int j = 0; j < KJ; ++j) kf[rr][j] = bf2f((uint16_t)kv[rr][j]);
          // the new position's key row comes from LDS (one key of the whole
          // range: a branch, so the other keys issue no LDS reads for it)
          if (__builtin_expect(k0 + c0 + hw + 16 * (b * SB + rr) == position, 0)) {
#pragma unroll
            for (int j = 0; j < KJ; ++j) kf[rr][j] = bf2f(s->khat[g * HD + l32 + 32 * j]);
          }
        }
        // each query head read from LDS once per batch of SB keys
#pragma unroll
        for (int hq = 0; hq < HPK; ++hq) {
          const float* qh = s->qhat + hq * HD + l32 * KJ;
          float qv[KJ];
#pragma unroll
          for (int j = 0; j < KJ; ++j) qv[j] = qh[j];
          // the two keys' trees at once: key 0's total in lane 0, key 1's in
          // lane 16 of the half wave
          static_assert(SB == 2, "paired score trees");
          float x[SB];
#pragma unroll
          for (int rr = 0; rr < SB; ++rr) {
            x[rr] = 0.0f;
#pragma unroll
            for (int j = 0; j < KJ; ++j) x[rr] += qv[j] * kf[rr][j];
          }
          const float tot = tree32_pair(x[0], x[1]);
          const int kk = hw + 16 * (b * SB + (l32 >> 4));  // sub-chunk relative
          if ((l32 & 15) == 0 && kk < sn) s->p[hq][kk] = tot * a.attn_scale;
        }
      };
      const int nb = (sn + 16 * SB - 1) / (16 * SB);
      uint32_t ka[SB][KJ], kb[SB][KJ];
      load_keys(ka, 0);
      int b = 0;
#pragma unroll 1
      for (; b + 1 < nb; b += 2) {
        load_keys(kb, b + 1);
        score_keys(ka, b);
        load_keys(ka, min(b + 2, nb - 1));
        score_keys(kb, b + 1);
      }
      if (b < nb) score_keys(ka, b);
      __syncthreads();
      clk.lap(1);
      // per query head (wave hq), groups of 32 tiles: tile maxima, the running
      // maximum (carried from the previous tiles of the range),
      // alpha_t = exp(m_{t-1} - m_t) (m_{-1} = -inf), p = exp(s - m_t)
      if (m.wave < HPK) {
        const int hq = m.wave;
        float carry = s->mr[hq];
#pragma unroll 1
        for (int tg = 0; tg < snt; tg += 32) {
          const int t = tg + (m.lane >> 1), kb4 = 8 * t + 4 * (m.lane & 1);
          float sv[4], mt = ninf;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            sv[j] = kb4 + j < sn ? s->p[hq][kb4 + j] : ninf;
            mt = fmaxf(mt, sv[j]);
          }
          mt = fmaxf(mt, __shfl_xor(mt, 1, 64));
          float run = mt;
#pragma unroll
          for (int d = 2; d < 64; d <<= 1) {
            const float o = __shfl_up(run, d, 64);
            if (m.lane >= d) run = fmaxf(run, o);
          }
          run = fmaxf(run, carry);
          float prev = __shfl_up(run, 2, 64);
          if (m.lane < 2) prev = carry;
          if (t < snt) {
            if (!(m.lane & 1)) s->alpha[hq][t] = hexp(prev - run);
#pragma unroll
            for (int j = 0; j < 4; ++j) s->p[hq][kb4 + j] = kb4 + j < sn ? hexp(sv[j] - run) : 0.0f;
          }
          const int last = min(snt - tg, 32) - 1;
          carry = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, run), 2 * last));
        }
        if (m.lane == 0) s->mr[hq] = carry;
      }
      __syncthreads();
      clk.lap(2);
      // V passes: the pass's rows into LDS, the next pass requested, then the
      // chains over the pass's tiles
      auto consume = [&](int q) {
        const int ta = 4 * q, tz = min(snt, ta + 4);
        if (chains) {
#pragma unroll 1
          for (int t = ta; t < tz; ++t) {
            float v0[8], v1[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
              const uint32_t pr = reinterpret_cast<const uint32_t*>(s->v[8 * (t - ta) + j])[cp];
              v0[j] = lo2f(pr);
              v1[j] = hi2f(pr);
            }
#pragma unroll
            for (int h = 0; h < 2; ++h) {
              const int hq = 2 * hp + h;
              const float al = s->alpha[hq][t];
              const f32x4 pa = *reinterpret_cast<const f32x4*>(&s->p[hq][8 * t]);
              const f32x4 pb = *reinterpret_cast<const f32x4*>(&s->p[hq][8 * t + 4]);
              const float pv[8] = {pa.x, pa.y, pa.z, pa.w, pb.x, pb.y, pb.z, pb.w};
              float x0 = acc[h][0] * al, x1 = acc[h][1] * al;
#pragma unroll
              for (int j = 0; j < 8; ++j) {
                x0 = x0 + pv[j] * v0[j];
                x1 = x1 + pv[j] * v1[j];
              }
              acc[h][0] = x0;
              acc[h][1] = x1;
            }
          }
        }
        if (m.tid < HPK) {
#pragma unroll 1
          for (int t = ta; t < tz; ++t) {
            const float al = s->alpha[m.tid][t];
            const f32x4 pa = *reinterpret_cast<const f32x4*>(&s->p[m.tid][8 * t]);
            const f32x4 pb = *reinterpret_cast<const f32x4*>(&s->p[m.tid][8 * t + 4]);
            den = den * al;
            den = den + pa.x; den = den + pa.y; den = den + pa.z; den = den + pa.w;
            den = den + pb.x; den = den + pb.y; den = den + pb.z; den = den + pb.w;
          }
        }
      };
#pragma unroll 1
      for (int q0 = 0; q0 < np; q0 += kFlashDepth) {
#pragma unroll
        for (int d = 0; d < kFlashDepth; ++d) {
          const int q = q0 + d;
          if (q < np) {
            put(ring[d]);
            __syncthreads();
            fetch(ring[d], q + kFlashDepth);
            consume(q);
            __syncthreads();
          }
        }
      }
      clk.lap(3);
    }
    // partial words of each query head of the group
    if (chains) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        uint64_t* w = Ly.x_scores + ((size_t)(g * HPK + 2 * hp + h) * kSplitRanges + r) * FW;
        word_store(w + 2 + 2 * cp, fbits(acc[h][0]), m.tag);
        word_store(w + 3 + 2 * cp, fbits(acc[h][1]), m.tag);
      }
    }
    if (m.tid < HPK) {
      uint64_t* w = Ly.x_scores + ((size_t)(g * HPK + m.tid) * kSplitRanges + r) * FW;
      word_store(w, fbits(s->mr[m.tid]), m.tag);
      word_store(w + 1, fbits(den), m.tag);
    }
    __syncthreads();
    clk.lap(3);
  }
  clk.flush(tb, nitems);
}

template <class S>
__device__ __forceinline__ void phase_merge(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, CHUNKS = HD / kValueChannels, ITEMS = S::Q * CHUNKS, FW = flash_words<S>();
  constexpr int RW = 2 + kValueChannels;  // words of one range taken: m, den, the chunk's channels
  const int64_t keys = (int64_t)G(a.params)[0] + 1;
  const int tiles = (int)((keys + 7) >> 3);
  const int rtiles = (tiles + kSplitRanges - 1) / kSplitRanges;
  const int nranges = (tiles + rtiles - 1) / rtiles;
  float* f = reinterpret_cast<float*>(m.big);  // [ranges][RW]
  float* wr = f + kSplitRanges * RW;           // w_r per range
  static_assert((kSplitRanges * (RW + 1)) * 4 <= kLdsBigBytes, "merge LDS");
  constexpr int PW = (kSplitRanges * RW + kMT - 1) / kMT;
  const float ninf = bitsf(0xff800000u);
#pragma unroll 1
  for (int slot = m.bid; slot < ITEMS; slot += m.grid) {
    const int head = slot / CHUNKS, c0 = (slot - head * CHUNKS) * kValueChannels;
    const uint64_t* base = Ly.x_scores + (size_t)head * kSplitRanges * FW;
    uint32_t gate_word = 0;
    if (m.wave == 0 && m.lane < kValueChannels / 2)
      gate_word = poll_one(m, Ly.x_proj + ((head * 2 * HD + HD + c0) >> 1) + m.lane);
    // every range's words at once
    poll_words<PW>(m, nranges * RW, [&](int i) {
      const int r = i / RW, k = i - r * RW;
      return base + (size_t)r * FW + (k < 2 ? k : c0 + k);
    }, reinterpret_cast<uint32_t*>(f));
    if (m.wave == 0) {
      float top = ninf;
      for (int r = m.lane; r < nranges; r += 64) top = fmaxf(top, f[r * RW]);
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) top = fmaxf(top, __shfl_xor(top, d, 64));
      for (int r = m.lane; r < nranges; r += 64) wr[r] = hexp(f[r * RW] - top);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
      float A = 0.0f, D = 0.0f;
      if (m.lane < kValueChannels) {
        // ranges in ascending order; each batch of 8 ranges' LDS reads is
        // issued before its sums, so the chains do not wait on every read
        int i = 0;
#pragma unroll 1
        for (; i + 8 <= nranges; i += 8) {
          float w8[8], d8[8], a8[8];
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            w8[k] = wr[i + k];
            d8[k] = f[(i + k) * RW + 1];
            a8[k] = f[(i + k) * RW + 2 + m.lane];
          }
#pragma unroll
          for (int k = 0; k < 8; ++k) {
            D = D + d8[k] * w8[k];
            A = A + a8[k] * w8[k];
          }
        }
        for (; i < nranges; ++i) {
          const float w = wr[i];
          D = D + f[i * RW + 1] * w;
          A = A + f[i * RW + 2 + m.lane] * w;
        }
      }
      const uint32_t gw = __shfl((int)gate_word, m.lane >> 1, 64);
      const uint16_t gb = (m.lane & 1) ? (uint16_t)(gw >> 16) : (uint16_t)(gw & 0xffffu);
      uint16_t y = 0;
      if (m.lane < kValueChannels) y = f2bf(rbf(A / D) * sigmoid(bf2f(gb)));
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
// wave per batch; a row streams in pieces of PIECE quads per lane,
// double-buffered, so the accumulation stays in reference order.
template <class S>
__device__ __forceinline__ void phase_head(const MegaArgs* pa, uint32_t tag) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int H = S::H, V = S::V, PER_LANE = (S::QH + 7) / 8;
  constexpr int PIECE = PER_LANE < 8 ? PER_LANE : 8, PIECES = (PER_LANE + PIECE - 1) / PIECE;
  static_assert(PIECES * PIECE == PER_LANE && S::QH % 8 == 0, "vocabulary pieces");
  constexpr int GROUPS = V / 8;  // 8-row groups; group gs + nw*b is this wave's batch b
  const int q = m.lane & 7, g = m.lane >> 3;
  const int nbatches = m.gs < GROUPS ? (GROUPS - 1 - m.gs) / m.nw + 1 : 0;
  const int steps = nbatches * PIECES;
  const uint32_t lane_off = (uint32_t)g * (uint32_t)H * 2u + (uint32_t)q * 16u;
  // piece t = (batch t / PIECES, piece t % PIECES); the group base address is
  // uniform, quad q + 8(pc*PIECE + j) of the lane's row is at byte 16q + 128(pc*PIECE + j)
  auto load_piece = [&](u32x4* buf, int t) {
    const int b = t / PIECES, pc = t - b * PIECES;
    const int grp = steps > 0 ? m.gs + m.nw * b : 0;  // a wave without groups reads group 0 (unused)
    const uint16_t* w = a.head + (size_t)(grp * 8) * H + pc * PIECE * 64;
#pragma unroll
    for (int j = 0; j < PIECE; ++j) buf[j] = ldq_at(w, lane_off + (uint32_t)j * 128u);
  };
  // Pieces past the wave's last one re-read the last (an L2 hit), so every
  // load is unconditional: the wait before a piece's products then leaves the
  // newer piece in flight (a conditional load makes the compiler drain them).
  const int last = steps > 0 ? steps - 1 : 0;
  u32x4 b0[PIECE], b1[PIECE];
  load_piece(b0, 0);
  f32x4 w0, w1;
  norm_weights<S>(m, a.out_norm, w0, w1);
  poll_words<(H / 2 + kMT - 1) / kMT>(m, H / 2, Span{a.x_final}, reinterpret_cast<uint32_t*>(m.xr));
  norm_row<S>(m, m.xr, w0, w1, a.eps);
  unsigned long long mine = 0ull;
  Quad acc;
  quad_zero(acc);
  auto consume = [&](const u32x4* buf, int t) {
    const int b = t / PIECES, pc = t - b * PIECES;
#pragma unroll
    for (int j = 0; j < PIECE; ++j) quad_acc(acc, m.xn[q + 8 * (pc * PIECE + j)], buf[j]);
    if (pc == PIECES - 1) {
      const float v = quad_tree<8>(acc);
      quad_zero(acc);
      const int row = (m.gs + m.nw * b) * 8 + g;
      if (q == 0) {
        const uint16_t bb = f2bf(v);
        G(a.logits)[row] = bb;
        const unsigned long long key = logit_key(bb, (uint32_t)row);
        mine = key > mine ? key : mine;
      }
    }
  };
  for (int t = 0; t < steps; t += 2) {
    load_piece(b1, min(t + 1, last));
    consume(b0, t);
    load_piece(b0, min(t + 2, last));
    if (t + 1 < steps) consume(b1, t + 1);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the re-reads, before the wave moves on
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

// Dynamic LDS of the step for shape S: the big area must also hold the
// down-projection staging.
template <class S>
constexpr int mega_big_bytes() {
  return DownLayout<S>::BYTES > kLdsBigBytes ? DownLayout<S>::BYTES : kLdsBigBytes;
}
template <class S>
constexpr int mega_lds_bytes() {
  return kLdsBig + mega_big_bytes<S>();
}

// Phase-trace stamps sit after the largest shape's LDS.
constexpr int kTraceLdsOffset = mega_lds_bytes<Shape35BA3B>();
static_assert(mega_lds_bytes<ShapeMiniMoE>() <= kTraceLdsOffset && mega_lds_bytes<ShapeTinyMoE>() <= kTraceLdsOffset,
              "trace offset");
__device__ __forceinline__ uint64_t* trace_lds() { return reinterpret_cast<uint64_t*>(mega_lds + kTraceLdsOffset); }

// Dynamic LDS the launch requests.
template <class S>
constexpr int mega_lds_request() {
#ifdef CQ35_PHASE_TRACE
  return kTraceLdsOffset + kTraceSlots * 8;
#else
  return mega_lds_bytes<S>();
#endif
}

__device__ __forceinline__ void trace_slot(int slot) {
#ifdef CQ35_PHASE_TRACE
  if (threadIdx.x == 0) reinterpret_cast<MegaMisc*>(mega_lds + kLdsMisc)->tslot = slot;
#else
  (void)slot;
#endif
}

template <class S>
__global__ __launch_bounds__(kMT) void k_decode_step(const MegaArgs* __restrict__ pa) {
  const uint32_t tag = (uint32_t)G(pa->params)[2];
  MegaMisc* misc = reinterpret_cast<MegaMisc*>(mega_lds + kLdsMisc);
  if (threadIdx.x == 0) {
    misc->abort = 0;
    misc->bid = blockIdx.x;
    misc->grid = gridDim.x;
    if (blockIdx.x == 0) {
      // cleared before any output of this block exists, so before any block
      // can reach the head
      __hip_atomic_store(G(pa->best), 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
  }
#ifdef CQ35_PHASE_TRACE
  for (int i = threadIdx.x; i < kTraceSlots; i += kMT) trace_lds()[i] = 0;
  if (threadIdx.x == 0) trace_lds()[kTraceStart] = __builtin_amdgcn_s_memrealtime();
#endif
  __syncthreads();
  const int L = pa->L;
  const MegaLayer* layers = pa->layers;
  ProjRegs<S> pr;
  issue_project<S, 0, kPairsEarly>(pa, layers, pr);
  for (int l = 0; l < L; ++l) {
    const MegaLayer* ly = layers + l;
    const int tb = l * kTraceLayerSlots;  // phase p: done at tb + 2p, inputs in at tb + 2p + 1
#ifdef CQ35_PHASE_TRACE
    if (threadIdx.x == 0) misc->tbase = tb;
#endif
    trace_slot(tb + 1);
    phase_project<S>(pa, tag, ly, l, pr);
    trace_max(tb + 0);
    if (phase_ptr(ly)->full != 0) {
      const int64_t keys = (int64_t)G(phase_ptr(pa)->params)[0] + 1;
      const int64_t split = phase_ptr(pa)->split_keys;
      trace_slot(tb + 3);
      if (split > 0 && keys > split) phase_flash<S>(pa, tag, ly, tb);
      else phase_scores<S>(pa, tag, ly);
      trace_max(tb + 2);
      trace_slot(tb + 5);
      if (split > 0 && keys > split) phase_merge<S>(pa, tag, ly);
      else phase_values<S>(pa, tag, ly, tb);
      trace_max(tb + 4);
      trace_slot(tb + 7);
      phase_outproj<S, S::QS>(pa, tag, ly);
    } else {
      trace_slot(tb + 3);
      phase_delta<S>(pa, tag, ly);
      trace_max(tb + 2);
      __syncthreads();
      trace_slot(tb + 7);
      phase_outproj<S, S::VS>(pa, tag, ly);
    }
    trace_max(tb + 6);
    trace_slot(tb + 9);
    phase_router<S>(pa, tag, ly);
    trace_max(tb + 8);
    trace_slot(tb + 11);
    phase_gate_up<S>(pa, tag, ly, l);
    trace_max(tb + 10);
    trace_slot(tb + 13);
    phase_down<S>(pa, tag, ly, l + 1 < L ? ly + 1 : nullptr, pr);
    trace_max(tb + 12);
  }
  trace_slot(kTraceHead + 2);
  phase_head<S>(pa, tag);
  trace_max(kTraceHead);
#ifdef CQ35_PHASE_TRACE
  __syncthreads();
  for (int i = threadIdx.x; i < kTraceSlots; i += kMT)
    pa->trace[(size_t)blockIdx.x * kTraceSlots + i] = trace_lds()[i];
#endif
}

}  // namespace cq35
