// Persistent one-launch decode step for the dense Qwen3.5 shapes (no MoE):
// the same resident-grid design as k_decode_step (every block runs every
// phase; phases hand over tagged 64-bit words), with the dense model's own
// orders:
//   * projections in S32 order (qwen35.rs dense path: simt.hex:400-410),
//     alpha and beta included, over the input row normalised per block;
//   * the Gated DeltaNet head step and the output projection of mega.h;
//   * staged attention (qwen35.rs:722-790 over attention.hex:71-92 and
//     qwen35_attention.hex:2-177, 258-393) as two phases: scalar-order
//     scores of every (query head, key), then per (head, channel chunk) the
//     head's softmax (a 256-partial maximum and the adjacent-pair sum over
//     the keys) and the context (eight interleaved chains per channel, the
//     sigmoid gate);
//   * the SwiGLU FFN: dual S256 gate/up (qwen3.fused.gate,
//     simt.hex:539-646) and the S64 down projection with the residual.
// Capacity is bounded (kDenseKeys) by the softmax, which holds a head's
// scores in LDS; longer sessions use the per-kernel path.
#pragma once

#include "mega.h"

namespace cq35 {

// Largest session capacity of the dense persistent step: a head's scores
// (F32) and 64-key nodes fit the big LDS area and its BF16 probabilities the
// polled-word area.
constexpr int kDenseKeys = 8064;
constexpr int kDenseFfnRows = 3;  // SwiGLU rows per wave

// Dense model shapes the persistent step is compiled for. Widths follow
// ModelConfig (src/spec.rs:33-62).
template <int H_, int V_, int Q_, int KVH_, int HD_, int R_, int KH_, int KD_, int VH_, int VD_, int I_>
struct DenseShape {
  static constexpr int H = H_, V = V_, Q = Q_, KVH = KVH_, HD = HD_, R = R_, KH = KH_, KD = KD_, VH = VH_,
                       VD = VD_, I = I_;
  static constexpr int KS = KH * KD, VS = VH * VD, QKV = 2 * KS + VS, QS = Q * HD, KVS = KVH * HD;
  static constexpr int QH = H / 8;
  static constexpr int NQA = (QH + 63) / 64;
  static constexpr bool kDense = true;
  static_assert(H % 64 == 0 && H <= 2048, "hidden width");
  static_assert(KD % 32 == 0 && KD <= 128 && VD <= 128 && VD % 4 == 0 && VH % 2 == 0, "DeltaNet head dims");
  static_assert(VH >= KH, "value heads");
  static_assert(HD == 64 || HD == 128 || HD == 256, "attention head dim");
  static_assert(Q <= 8 && Q % KVH == 0 && KVH <= 2 && R <= HD && R % 2 == 0, "attention heads");
  static_assert(QS <= 4096 && VS <= 4096 && I % 128 == 0 && I <= 8192, "widths");
  static_assert(V % 8 == 0, "vocabulary in groups of 8 rows");
};
// qwen35-2b, qwen35-0.8b (src/spec.rs:121-151) and the two reduced dense test shapes.
using ShapeDense2B = DenseShape<2048, 248320, 8, 2, 256, 64, 16, 128, 32, 128, 6144>;
using ShapeDense08B = DenseShape<1024, 248320, 8, 2, 256, 64, 16, 128, 16, 128, 3584>;
using ShapeDenseMini = DenseShape<512, 8192, 4, 2, 256, 64, 2, 128, 4, 128, 1408>;
using ShapeDenseTiny = DenseShape<256, 4096, 4, 1, 64, 16, 4, 32, 8, 32, 768>;

// ------------------------------------------------- phase: S32 projection

// Normalised input row x the layer's projection segments in S32 order: 8
// lanes per row (physical lane q holds reference lanes 4q..4q+3 and visits
// quads q, q + 8, ...), 8 rows per wave per round, row 8(gs + nw k) + g for
// lane group g (gs: waves interleaved across blocks); the group's tree (quad_tree<8>), rows 2p and 2p+1 packed into
// one word by the even group. The round's weights are issued before the
// input row is polled.
template <class S>
__device__ __forceinline__ void phase_project32(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly, int l) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  constexpr int NQ = S::QH / 8;
  static_assert(S::QH % 8 == 0, "S32 rows");
  const int rows = Ly.seg_rows[0] + Ly.seg_rows[1] + Ly.seg_rows[2] + Ly.seg_rows[3];
  const int q = m.lane & 7, g = m.lane >> 3;
  const int rounds = (rows + 8 * m.nw - 1) / (8 * m.nw);
  u32x4 wv[NQ];
  // a wave whose eight rows all lie past the end loads and computes nothing
  // (uniform per wave); the wave holding the end clamps its last rows
  auto issue = [&](int k) {
    if (8 * (m.gs + m.nw * k) >= rows) {
#pragma unroll
      for (int j = 0; j < NQ; ++j) wv[j] = u32x4{0u, 0u, 0u, 0u};
      return;
    }
    const int row = min(8 * (m.gs + m.nw * k) + g, rows - 1);
    const uint16_t* w = seg_row(Ly, row, S::H);
#pragma unroll
    for (int j = 0; j < NQ; ++j) wv[j] = ldq_at(w, (uint32_t)(q + 8 * j) * 16u);
  };
  issue(0);
  f32x4 w0, w1;
  norm_weights<S>(m, Ly.in_norm, w0, w1);
  load_hidden<S>(m, Ly.x_h, m.xr, l == 0);
  norm_row<S>(m, m.xr, w0, w1, m.a.eps);
  trace_mark(kMarkProjectNormed);
#pragma unroll 1
  for (int k = 0; k < rounds; ++k) {
    if (k > 0) issue(k);
    if (8 * (m.gs + m.nw * k) >= rows) continue;  // uniform per wave
    const int row = 8 * (m.gs + m.nw * k) + g;
    Quad acc;
    quad_zero(acc);
#pragma unroll
    for (int j = 0; j < NQ; ++j) quad_acc(acc, m.xn[q + 8 * j], wv[j]);
    const float v = quad_tree<8>(acc);
    const uint32_t b = f2bf(v);
    const uint32_t other = (uint32_t)__shfl_down((int)b, 8, 64);
    if (q == 0 && (g & 1) == 0 && row < rows) word_store(Ly.x_proj + (row >> 1), pack_bf((uint16_t)b, (uint16_t)other), m.tag);
  }
}

// ------------------------------------- phase: staged attention scores

struct DenseScoreLds {
  float rope[256];
  float normed[kMW][256];
  float qhat[8 * 256];  // prepare_heads' lane-major query heads
  float qnat[8 * 256];  // the same in channel order for the serial chains
  uint16_t khat[2 * 256];
  int heads[32];
  int nheads;
};
static_assert(sizeof(DenseScoreLds) <= kLdsBigBytes, "dense score LDS");
static_assert(offsetof(DenseScoreLds, qnat) % 16 == 0, "dense score LDS alignment");

// Every block prepares all query and key heads (head RMS with the
// adjacent-pair tree, neox RoPE; full_prepare.hex:3-82); block 0 appends the
// new position's K and V to the cache. Then one (query head, 64-key chunk)
// per wave, item i on wave i / grid of block i % grid (spread over the CUs,
// so none streams more than a few key rows; the lanes share the query head,
// an LDS broadcast): score = bf16(serial chain over the head's channels,
// element 0 first, x scale) (staged_score), one tagged word each in
// x_scores[head][key]. The new position's key row comes from LDS.
template <class S>
__device__ __forceinline__ void phase_dense_scores(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, Q = S::Q, KVH = S::KVH, HPK = Q / KVH, KJ = HD / 32, RH = S::R / 2, VPL = HD / 64;
  constexpr int QW = Q * HD / 2, KW = S::KVS / 2;
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  DenseScoreLds* s = reinterpret_cast<DenseScoreLds*>(m.big);
  float qw_[VPL], kw_[VPL];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    qw_[i] = G(Ly.qnorm)[VPL * m.lane + i];
    kw_[i] = G(Ly.knorm)[VPL * m.lane + i];
  }
  const float freq = G(a.freq)[min(m.tid, RH - 1)];
  // query parts of every head ([q(HD) | gate(HD)] per head), key heads, value heads
  const uint64_t* proj = Ly.x_proj;
  auto index = [&](int i) -> int {
    if (i < QW) {
      const int hq = i / (HD / 2), c = i - hq * (HD / 2);
      return hq * HD + c;
    }
    return S::QS + (i - QW);  // key heads, then value heads
  };
  poll_words<(QW + 2 * KW + kMT - 1) / kMT>(m, QW + 2 * KW, [&](int i) { return proj + index(i); }, m.vec);
  const uint16_t* in16 = reinterpret_cast<const uint16_t*>(m.vec);
  const int chunks = (int)((keys + 63) >> 6);
  const int witems = Q * chunks;
  // the heads this block needs: the query heads of its items, the key head
  // of an item holding the new position (a head's last chunk) and, on block
  // 0, every key head (the cache append)
  if (m.tid == 0) {
    int nh = 0;
    auto add = [&](int hh) {
      bool seen = false;
      for (int i = 0; i < nh; ++i) seen |= s->heads[i] == hh;
      if (!seen) s->heads[nh++] = hh;
    };
    for (int w = 0; w < kMW; ++w) {
      const int wi = m.bid + m.grid * w;
      if (wi >= witems) break;
      const int hq = wi / chunks;
      add(hq);
      if (wi - hq * chunks == chunks - 1) add(Q + hq / HPK);
    }
    if (m.bid == 0)
      for (int g = 0; g < KVH; ++g) add(Q + g);
    s->nheads = nh;
  }
  if (m.tid < RH) {
    float sn, cs;
    sincos_q((float)(uint32_t)position * freq, &sn, &cs);
    s->rope[m.tid] = cs;
    s->rope[RH + m.tid] = sn;
  }
  __syncthreads();
  const int nheads = s->nheads;
  prepare_heads<S>(m, s, nheads, qw_, kw_, [&](int hh) {
    return hh < Q ? in16 + hh * HD : in16 + 2 * QW + (hh - Q) * HD;
  }, [&](int hh) { return hh; });
  for (int i = m.tid; i < nheads * HD; i += kMT) {
    const int hq = s->heads[i / HD], c = i % HD;
    if (hq < Q) s->qnat[hq * HD + c] = s->qhat[hq * HD + (c & 31) * KJ + (c >> 5)];
  }
  if (m.bid == 0 && m.tid < S::KVS) {
    G(a.cache)[Ly.key_base + position * S::KVS + m.tid] = s->khat[m.tid];
    G(a.cache)[Ly.value_base + position * S::KVS + m.tid] = in16[2 * QW + S::KVS + m.tid];
  }
  __syncthreads();
  trace_mark(kMarkDeltaConv);  // full layers of the dense step: heads prepared
#pragma unroll 1
  for (int wi = m.bid + m.grid * m.wave; wi < witems; wi += m.grid * kMW) {  // uniform per wave
    const int hq = wi / chunks;
    const int64_t key = (int64_t)(wi - hq * chunks) * 64 + m.lane;
    const int g = hq / HPK;
    const float* qf = s->qnat + hq * HD;
    if (key < keys) {
      float acc;
      if (key == position) {
        acc = 0.0f;
        for (int c = 0; c < HD; ++c) acc += qf[c] * bf2f(s->khat[g * HD + c]);
      } else {
        acc = staged_score(a.cache + Ly.key_base + key * S::KVS + g * HD, qf, HD);
      }
      word_store(Ly.x_scores + (int64_t)hq * a.cap + key, fbits(rbf(acc * a.attn_scale)), m.tag);
    }
  }
}

// --------------------------------- phase: staged attention softmax + context

constexpr int kAttendChannels = 8;   // channels per item
constexpr int kAttendKeys = 1024;    // keys staged per chunk

// Item (query head, 8-channel chunk), Q * HD / 8 items over the blocks. The
// item's value slices (16 bytes per key) for its first two chunks are
// requested first; then the block polls the head's scores into LDS and runs
// the softmax (qwen35_attention.hex:258-393): the maximum (exact in any
// order: wave reductions), the adjacent-pair sum over the keys (its first
// six levels, pairs within a 64-key group, across the lanes of a wave; the
// rest over the 64-key nodes in LDS; the same additions as the
// level-by-level loop) and p = bf16(exp(s - max) / sum) into LDS. Then the
// context (qwen35_attention.hex:2-177): per channel eight chains over keys
// r, r + 8, ... in order (the tail padded with + 0) on threads tid < 64
// (chain tid / 8, channel tid % 8), combined ((a0+a4)+(a2+a6))+
// ((a1+a5)+(a3+a7)), then bf16(bf16(sum) * sigmoid(gate)) (qwen35.hex:
// 207-222). Value slices are staged kAttendKeys keys at a time; the new
// position's slice comes from the projection words. Every item of a head
// repeats the head's softmax: it costs less than another exchange.
template <class S>
__device__ __forceinline__ void phase_dense_attend(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  const CQ35_CONST MegaArgs& a = m.a;
  constexpr int HD = S::HD, Q = S::Q, HPK = Q / S::KVH, CH = kAttendChannels, KC = kAttendKeys;
  constexpr int ITEMS = Q * HD / CH;
  constexpr int VPT = KC / kMT;  // 16-byte slices per thread per chunk
  constexpr int KPT = (kDenseKeys + kMT - 1) / kMT;
  static_assert(KC % kMT == 0 && 2 * KC * CH * 2 + 8 * CH * 4 <= kLdsBigBytes, "attend staging");
  static_assert((kDenseKeys + kDenseKeys / 64) * 4 <= kLdsBigBytes && kDenseKeys * 2 <= 4096 * 4, "attend LDS");
  const int64_t position = (int64_t)G(a.params)[0];
  const int64_t keys = position + 1;
  const int64_t steps = (keys + 7) >> 3;
  const int nchunks = (int)((8 * steps + KC - 1) / KC);
  const float ninf = bitsf(0xff800000u);
  const int r = m.tid >> 3, x = m.tid & 7;
#pragma unroll 1
  for (int item = m.bid; item < ITEMS; item += m.grid) {
    const int hq = item / (HD / CH), c0 = (item - hq * (HD / CH)) * CH;
    const int g = hq / HPK;
    const uint16_t* vb = a.cache + Ly.value_base + (int64_t)g * HD + c0;
    u32x4 vr[2][VPT];
    auto fetch = [&](u32x4 (&dst)[VPT], int ch) {
      const int64_t k0 = (int64_t)ch * KC;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int64_t key = min(k0 + m.tid + kMT * i, position - 1 >= 0 ? position - 1 : 0);
        dst[i] = *G(reinterpret_cast<const u32x4*>(vb + key * S::KVS));
      }
    };
    fetch(vr[0], 0);
    fetch(vr[1], min(1, nchunks - 1));
    // the gate channels and the new position's value slice (4 words each)
    uint32_t extra = 0;
    if (m.tid < CH)
      extra = poll_one(m, m.tid < CH / 2 ? Ly.x_proj + ((hq * 2 * HD + HD + c0) >> 1) + m.tid
                                         : Ly.x_proj + ((2 * S::QS + S::KVS + g * HD + c0) >> 1) + (m.tid - CH / 2));
    // softmax of head hq
    float* sc = reinterpret_cast<float*>(m.big);
    float* nodes = sc + kDenseKeys;
    poll_words_upto<KPT>(m, (int)keys, Span{Ly.x_scores + (int64_t)hq * a.cap}, reinterpret_cast<uint32_t*>(sc));
    uint16_t* p16 = reinterpret_cast<uint16_t*>(m.vec);
    uint32_t* extra_lds = reinterpret_cast<uint32_t*>(m.misc->scalars);
    if (m.tid < CH) extra_lds[m.tid] = extra;
    const int nk = (int)keys;
    float sv[KPT];
    float mx = ninf;
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int kk = m.tid + kMT * j;
      sv[j] = kk < nk ? sc[kk] : ninf;
      mx = fmaxf(mx, sv[j]);
    }
    // wave maximum in lane 0 (its DPP reads never leave its rows)
    mx = fmaxf(mx, lane_down<32>(mx));
    mx = fmaxf(mx, lane_down<16>(mx));
    mx = fmaxf(mx, lane_down<8>(mx));
    mx = fmaxf(mx, lane_down<4>(mx));
    mx = fmaxf(mx, lane_down<2>(mx));
    mx = fmaxf(mx, lane_down<1>(mx));
    if (m.lane == 0) m.misc->red[m.wave] = mx;
    __syncthreads();
    float maximum = m.misc->red[0];
#pragma unroll
    for (int w = 1; w < kMW; ++w) maximum = fmaxf(maximum, m.misc->red[w]);
    // pair sums within each 64-key group: level d adds key k + d into key k
    // (k a multiple of 2d) when k + d exists
    auto group_levels = [&](float e, int kk, int limit) {
      float o;
      o = lane_down<1>(e);  if ((m.lane & 1) == 0 && kk + 1 < limit) e += o;
      o = lane_down<2>(e);  if ((m.lane & 3) == 0 && kk + 2 < limit) e += o;
      o = lane_down<4>(e);  if ((m.lane & 7) == 0 && kk + 4 < limit) e += o;
      o = lane_down<8>(e);  if ((m.lane & 15) == 0 && kk + 8 < limit) e += o;
      o = lane_down<16>(e); if ((m.lane & 31) == 0 && kk + 16 < limit) e += o;
      o = lane_down<32>(e); if (m.lane == 0 && kk + 32 < limit) e += o;
      return e;
    };
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int base = kMT * j + 64 * m.wave, kk = base + m.lane;
      if (base < nk) {  // uniform per wave
        const float e = group_levels(kk < nk ? hexp(sv[j] - maximum) : 0.0f, kk, nk);
        if (m.lane == 0) nodes[base >> 6] = e;
      }
    }
    __syncthreads();
    // levels 64 and up over the nodes (node n = keys 64n..), on wave 0: lane
    // l holds nodes l and l + 64; the same levels, then node 0 += node 64
    const int nn = (nk + 63) >> 6;
    static_assert(kDenseKeys <= 128 * 64, "two nodes per lane");
    if (m.wave == 0) {
      float v0 = m.lane < nn ? nodes[m.lane] : 0.0f;
      float v1 = m.lane + 64 < nn ? nodes[m.lane + 64] : 0.0f;
      v0 = group_levels(v0, m.lane, nn);
      v1 = group_levels(v1, m.lane + 64, nn);
      if (m.lane == 0) m.misc->red[0] = nn > 64 ? v0 + v1 : v0;
    }
    __syncthreads();
    const float den = m.misc->red[0];
#pragma unroll
    for (int j = 0; j < KPT; ++j) {
      const int kk = m.tid + kMT * j;
      if (kk < nk) p16[kk] = f2bf(hexp(sv[j] - maximum) / den);
    }
    __syncthreads();  // probabilities in; the score area becomes the value staging
    trace_mark(kMarkDeltaGates);  // full layers of the dense step: softmax done
    uint16_t(*vs)[KC][CH] = reinterpret_cast<uint16_t(*)[KC][CH]>(m.big);
    const uint32_t* vnw = extra_lds + CH / 2;  // the new value slice
    auto put = [&](int buf, const u32x4 (&src)[VPT], int ch) {
      const int64_t k0 = (int64_t)ch * KC;
#pragma unroll
      for (int i = 0; i < VPT; ++i) {
        const int idx = m.tid + kMT * i;
        const u32x4 v = k0 + idx == position ? u32x4{vnw[0], vnw[1], vnw[2], vnw[3]} : src[i];
        *reinterpret_cast<u32x4*>(&vs[buf][idx][0]) = v;
      }
    };
    put(0, vr[0], 0);
    __syncthreads();
    float acc = 0.0f;
#pragma unroll 1
    for (int ch = 0; ch < nchunks; ++ch) {
      const int buf = ch & 1;
      if (ch + 1 < nchunks && ch > 0) fetch(vr[(ch + 1) & 1], ch + 1);  // chunk 1 is already in flight
      if (m.tid < 64) {
        // chain r's keys k0 + 8 i + r; only the last step of all may be past the end
        const int k0 = ch * KC;
        const int n = min(KC / 8, (int)steps - k0 / 8);
        const bool last = ch == nchunks - 1;
        const int full = last ? n - 1 : n;
        const uint16_t* pc = p16 + k0 + r;
        const uint16_t* vc = &vs[buf][r][x];
#pragma unroll 8
        for (int i = 0; i < full; ++i) acc = acc + bf2f(pc[8 * i]) * bf2f(vc[8 * CH * i]);
        if (last) {
          const int kk = k0 + 8 * (n - 1) + r;
          const float pv = bf2f(p16[kk < (int)keys ? kk : 0]), vv = bf2f(vc[8 * CH * (n - 1)]);
          acc = acc + (kk < (int)keys ? pv * vv : 0.0f);
        }
      }
      if (ch + 1 < nchunks) put(buf ^ 1, vr[(ch + 1) & 1], ch + 1);
      __syncthreads();
    }
    trace_mark(kMarkDeltaState);  // full layers of the dense step: chains done
    float* part = reinterpret_cast<float*>(m.big + 2 * KC * CH * 2);
    if (m.tid < 64) part[r * CH + x] = acc;
    __syncthreads();
    if (m.tid < CH) {
      const int t = m.tid;
      const float sum = ((part[0 * CH + t] + part[4 * CH + t]) + (part[2 * CH + t] + part[6 * CH + t])) +
                        ((part[1 * CH + t] + part[5 * CH + t]) + (part[3 * CH + t] + part[7 * CH + t]));
      const uint32_t gw = extra_lds[t >> 1];
      const uint16_t gb = (uint16_t)((t & 1) ? (gw >> 16) : (gw & 0xffffu));
      const uint32_t y = f2bf(rbf(sum) * sigmoid(bf2f(gb)));
      const uint32_t other = (uint32_t)__shfl_down((int)y, 1, 64);
      if ((t & 1) == 0) word_store(Ly.x_mix + ((hq * HD + c0 + t) >> 1), pack_bf((uint16_t)y, (uint16_t)other), m.tag);
    }
    __syncthreads();
  }
}

// -------------------------------------------------- phase: SwiGLU gate/up

// Every block normalises the post-mixer row (post_attention_norm) into m.xn
// and keeps the raw row in m.xa for the down projection's residual. Wave
// slot gp takes rows gp + nw k (k < kDenseFfnRows; wave pairs interleaved
// across blocks): gate and up rows in S256 order
// (64 lanes, quads lane + 64 j), t = bf16(bf16(silu(bf16 g)) * bf16 u); even
// waves hold even rows and store the word of the pair.
template <class S>
__device__ __forceinline__ void phase_dense_gate_up(const MegaArgs* pa, uint32_t tag, const MegaLayer* ly) {
  const Mega m = make_mega(pa, tag);
  const CQ35_CONST MegaLayer& Ly = *phase_ptr(ly);
  constexpr int NQ = S::NQA, RG = kDenseFfnRows, H = S::H, QH = S::QH;
  // wave pairs (the two rows of an output word) interleaved across blocks
  const int gp = (((m.wave >> 1) * m.grid + m.bid) << 1) | (m.wave & 1);
  u32x4 gv[RG][NQ], uv[RG][NQ];
#pragma unroll
  for (int k = 0; k < RG; ++k) {
    if (gp + m.nw * k >= S::I) {  // no row (uniform per wave): nothing to load
#pragma unroll
      for (int j = 0; j < NQ; ++j) gv[k][j] = uv[k][j] = u32x4{0u, 0u, 0u, 0u};
      continue;
    }
    const int row = gp + m.nw * k;
    const uint16_t* wg = Ly.sgate + (size_t)row * H;
    const uint16_t* wu = Ly.sup + (size_t)row * H;
#pragma unroll
    for (int j = 0; j < NQ; ++j) {
      gv[k][j] = ldq_at(wg, (uint32_t)min(m.lane + 64 * j, QH - 1) * 16u);
      uv[k][j] = ldq_at(wu, (uint32_t)min(m.lane + 64 * j, QH - 1) * 16u);
    }
  }
  f32x4 w0, w1;
  norm_weights<S>(m, Ly.post_norm, w0, w1);
  poll_words<(H / 2 + kMT - 1) / kMT>(m, H / 2, Span{Ly.x_attn}, reinterpret_cast<uint32_t*>(m.xa));
  norm_row<S>(m, m.xa, w0, w1, m.a.eps);
  trace_mark(kMarkRouterNormed);
  uint16_t* odd = reinterpret_cast<uint16_t*>(m.big);  // [kMW / 2][RG]
  // the rows' total pairs (wave-uniform); the epilogues then run one per
  // lane, lane k taking row k
  float gs[RG], us[RG];
#pragma unroll
  for (int k = 0; k < RG; ++k) {
    const int row = gp + m.nw * k;
    gs[k] = us[k] = 0.0f;
    if (row < S::I) {  // uniform per wave
      Quad ga, ua;
      quad_zero(ga);
      quad_zero(ua);
#pragma unroll
      for (int j = 0; j < NQ; ++j)
        if (QH % 64 == 0 || m.lane + 64 * j < QH) {
          const u32x4 xq = m.xn[m.lane + 64 * j];
          quad_acc(ga, xq, gv[k][j]);
          quad_acc(ua, xq, uv[k][j]);
        }
      const float tot = quad_tree64_pair_end(ga, ua);  // gate total in lane 31, up total in lane 63
      gs[k] = lane_value(tot, 31);
      us[k] = lane_value(tot, 63);
    }
  }
  float gsum = 0.0f, usum = 0.0f;
#pragma unroll
  for (int k = 0; k < RG; ++k)
    if (m.lane == k) {
      gsum = gs[k];
      usum = us[k];
    }
  const uint16_t t = bf_mul(f2bf(silu(rbf(gsum))), f2bf(usum));  // row m.lane (lanes < RG)
  const int my_row = gp + m.nw * m.lane;
  if (m.lane < RG && my_row < S::I && (m.wave & 1)) odd[(m.wave >> 1) * RG + m.lane] = t;
  trace_mark(kMarkGateUpDone);
  __syncthreads();
  if (m.lane < RG && my_row < S::I && !(m.wave & 1))
    word_store(Ly.x_active + (my_row >> 1), pack_bf(t, odd[(m.wave >> 1) * RG + m.lane]), m.tag);
}

// ------------------------------------------------------------- the kernel

template <class S>
constexpr int dense_lds_bytes() {
  return kLdsBig + kLdsBigBytes;
}
static_assert(dense_lds_bytes<ShapeDense2B>() <= kTraceLdsOffset, "dense trace offset");

template <class S>
constexpr int dense_lds_request() {
#ifdef CQ35_PHASE_TRACE
  return kTraceLdsOffset + kTraceSlots * 8;
#else
  return dense_lds_bytes<S>();
#endif
}

// Phase slots of the dense step's trace: p0 project, p1 delta or scores,
// p3 softmax + context, p4 output projection, p5 gate/up, p6 down.
template <class S>
__global__ __launch_bounds__(kMT) void k_dense_step(const MegaArgs* __restrict__ pa) {
  const uint32_t tag = (uint32_t)G(pa->params)[2];
  MegaMisc* misc = reinterpret_cast<MegaMisc*>(mega_lds + kLdsMisc);
  if (threadIdx.x == 0) {
    misc->abort = 0;
    misc->bid = blockIdx.x;
    misc->grid = gridDim.x;
    if (blockIdx.x == 0) {
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
  for (int l = 0; l < L; ++l) {
    const MegaLayer* ly = layers + l;
    const int tb = l * kTraceLayerSlots;
#ifdef CQ35_PHASE_TRACE
    if (threadIdx.x == 0) misc->tbase = tb;
#endif
    trace_slot(tb + 1);
    phase_project32<S>(pa, tag, ly, l);
    trace_max(tb + 0);
    if (phase_ptr(ly)->full != 0) {
      trace_slot(tb + 3);
      phase_dense_scores<S>(pa, tag, ly);
      trace_max(tb + 2);
      __syncthreads();
      trace_slot(tb + 7);
      phase_dense_attend<S>(pa, tag, ly);
      trace_max(tb + 6);
      __syncthreads();
      trace_slot(tb + 9);
      phase_outproj<S, S::QS>(pa, tag, ly);
    } else {
      trace_slot(tb + 3);
      phase_delta<S>(pa, tag, ly);
      trace_max(tb + 2);
      __syncthreads();
      trace_slot(tb + 9);
      phase_outproj<S, S::VS>(pa, tag, ly);
    }
    trace_max(tb + 8);
    trace_slot(tb + 11);
    phase_dense_gate_up<S>(pa, tag, ly);
    trace_max(tb + 10);
    trace_slot(tb + 13);
    phase_outproj<S, S::I, true>(pa, tag, ly);
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
