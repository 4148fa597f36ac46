/*
 * CPU restatement of catena-models' Qwen3.5/3.6 token loop, used ONLY as the
 * parity checker and the CPU baseline. This is test infrastructure: nothing in
 * the shipped library links, loads or calls it.
 *
 * Every function restates the operation order and rounding points of the
 * reference Hex kernels (file:line citations are into hellas-ai/catena-models).
 * Arithmetic is plain IEEE binary32 with FMA contraction disabled
 * (build with -ffp-contract=off), matching numeric.hex:10.
 *
 * How each part is pinned (the reference itself cannot run here: its compiler
 * crate catena-lang is not in the tree and there is no Rust toolchain):
 *  - ox_f2bf / BF16 add and mul: RNE closed form over all exponent classes,
 *    and the bit-exact epilogues of the known-answer fixtures.
 *  - ox_exp: the reference's accuracy contract (tests/support/
 *    portable_exp.cpp:26-102: <= 1 ULP against float64, exact specials,
 *    NaN -> 0x7fc00000), with a planted-mistake check.
 *  - ox_sqrt / ox_softplus / ox_sincos: closed forms (Newton limit, log1p(e^x),
 *    sin/cos) at their documented accuracy.
 *  - ox_project, ox_residual_project, grouped projections, router, MoE down
 *    (S32 / S64 / S256 trees, split lo/hi accumulators, BF16 epilogues):
 *    bit-exact known answers from the generators of tests/qwen35_simt.rs
 *    (129-436), plus F32 random-dot fixtures that a wrong tree width fails.
 *  - ox_moe_gate_rows: within the reference test's own 1% bar
 *    (tests/qwen35_simt.rs:309-389).
 *  - conv, L2 norms, gated delta rule (BF16 and F32 state), gated RMSNorm,
 *    hidden and head RMS norms, RoPE (positions to 2^17), online and staged
 *    attention (up to 4100 keys): each function against a float64 formulation
 *    within 1-4 BF16 unit roundoffs (relative RMS), and each with planted
 *    mistakes (ox_set_plant: rotation pairing / sign / frequency exponent,
 *    q/k norm swap, conv tap order, delta scale, prediction decay, key-head
 *    map, L2 span, gated mean, attention scale, GQA map, norm weights) that
 *    miss by 12x the tolerance or more (tests/test_oracle_pins.py).
 *  - ox_step: every cached K/V row and DeltaNet state after a short decode,
 *    and the logits, new rows and state of one step at position 5000 from an
 *    imported state, against a float64 textbook model within 10-12 U, the
 *    same planted mistakes missing by 3x or more; logits of whole prompts
 *    within 0.15 relative RMS. The exact reduction orders inside these
 *    functions (D32, AP, SER, dense-staged, CONV) are restated from the Hex
 *    text and no reference-held vector fixes them: those orders are pinned
 *    to tolerance only.
 *  - parity unpinned: stdlib.math.round_to_u32 at exact .5 ties (taken as
 *    ties away from zero), f32.max with NaN operands, bf16x2 low/high order
 *    (taken as little-endian), core.fold.bounded order (taken as ascending).
 *    Their definitions live in catena-lang, which is absent.
 */
#ifndef CQ35_ORACLE_H
#define CQ35_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Field-for-field the subset of ModelConfig (src/spec.rs:33-62) the token loop
 * reads. moe != 0 selects ModelArchitecture::Qwen35Moe. */
typedef struct ox_config {
  int32_t moe;
  int32_t vocab;
  int32_t hidden;
  int32_t intermediate;     /* dense FFN width, or per-expert width (MoE) */
  int32_t layers;
  int32_t q_heads;
  int32_t kv_heads;
  int32_t head_dim;
  int32_t rope_dim;
  float eps;
  float theta;
  int32_t experts;
  int32_t top_k;
  int32_t shared_intermediate;
  int32_t full_interval;
  int32_t key_heads;        /* linear_group_count */
  int32_t key_dim;          /* linear_state_size */
  int32_t value_heads;      /* linear_time_step_rank */
  int32_t value_dim;        /* linear_inner_size / value_heads */
  int32_t tied;
} ox_config;

enum { OX_BF16 = 0, OX_F32 = 1 };

/* Weight ABI: the ordered list of src/spec.rs:443-712 (weight_specs). */
int64_t ox_weight_count(const ox_config* c);
/* dtype (OX_BF16/OX_F32), rows, cols (cols==1 for vectors), kind (see oracle.c). */
int ox_weight_info(const ox_config* c, int64_t index, int32_t* dtype, int64_t* rows,
                   int64_t* cols, int32_t* kind);

/* Numerics (numeric.hex). */
float ox_exp(float x);
float ox_silu(float x);
float ox_sigmoid(float x);
float ox_softplus(float x);
float ox_sqrt(float x);
void ox_sincos(float angle, float* sine, float* cosine);
uint16_t ox_f2bf(float x);
float ox_bf2f(uint16_t b);

/* Split-pair dot with a halving tree of the given width (tests/qwen35_simt.rs:99-116). */
float ox_dot_width(const uint16_t* x, const uint16_t* w, int64_t pairs, int width);
float ox_dot_width_f32w(const uint16_t* x, const float* w, int64_t pairs, int width);
/* B256 single-accumulator dot of the batched prefill (batch_projection.hex:4-18). */
float ox_dot_b256(const uint16_t* x, const uint16_t* w, int64_t pairs);

/* Synthetic weights: the deterministic generator shared (as a specification)
 * with the GPU library. Fills one tensor of the weight ABI. */
void ox_fill_tensor(const ox_config* c, uint64_t seed, int64_t index, void* dst);
uint64_t ox_mix64(uint64_t x);

/* Model (weights held by reference; the caller owns them). */
typedef struct ox_model ox_model;
ox_model* ox_model_create(const ox_config* c, void* const* weights);
void ox_model_free(ox_model* m);

/* Session = the reference's opaque state (state_init_*.hex) in the reference
 * layout: cache BF16 [KV | per-layer conv history + recurrent], workspace F32
 * shadow [layers * recurrent]. */
typedef struct ox_session ox_session;
ox_session* ox_session_create(const ox_model* m, int64_t capacity);
void ox_session_free(ox_session* s);
int64_t ox_cache_elements(const ox_config* c, int64_t capacity);
uint16_t* ox_session_cache(ox_session* s);
float* ox_session_shadow(ox_session* s);

/* One `qwen3` call (src/qwen/qwen35.rs:1466-1650): processes tokens at
 * positions start..start+n and returns the greedy token of the last one.
 * Returns 0 on success, <0 on invalid input, -9 for the batched (n>=2,
 * key_dim==128) prefill path, which this restatement does not cover. */
int ox_step(ox_session* s, const uint64_t* tokens, int64_t n, int64_t start,
            uint64_t* next_token, uint16_t* logits);

/* Decode attention (online, MoE) over more than `keys` cached keys runs as
 * at most 128 ranges of equal tile counts, each with its own online
 * recurrence, merged in ascending order (this build's long-context mode, tolerance-level against
 * the reference's single chain); 0 keeps the single chain at every length.
 * Default OX_SPLIT_KEYS_DEFAULT, the GPU library's default. */
#define OX_SPLIT_KEYS_DEFAULT 8192
void ox_session_set_split_keys(ox_session* s, int64_t keys);

/* Router diagnostics of the last MoE step: ids[layer*top_k + j]. */
const int64_t* ox_session_last_ids(const ox_session* s);

void ox_set_threads(int n);

/* Planted mistakes for the pinning tests (never set in normal use): each
 * switches one restated function to a plausible wrong variant. */
enum {
  OX_PLANT_NONE = 0,
  OX_PLANT_ROPE_PAIRING = 1,     /* interleaved (2i, 2i+1) rotation pairs */
  OX_PLANT_ROPE_SIGN = 2,        /* rotation by -angle */
  OX_PLANT_ROPE_FREQ_HD = 3,     /* frequency exponent over head_dim, not rope_dim */
  OX_PLANT_QK_NORM_SWAP = 4,     /* q heads normed with k_norm and vice versa */
  OX_PLANT_CONV_TAP_ORDER = 5,   /* conv taps applied in reverse order */
  OX_PLANT_DELTA_SCALE = 6,      /* output dot without 1/sqrt(key_dim) */
  OX_PLANT_L2_WHOLE = 7,         /* L2 norm over all heads at once */
  OX_PLANT_GATED_SUM = 8,        /* gated RMS from the sum, not the mean */
  OX_PLANT_ATTN_SCALE = 9,       /* scores without 1/sqrt(head_dim) */
  OX_PLANT_GQA_MAP = 10,         /* query head h reads KV head h % kv_heads */
  OX_PLANT_NORM_WEIGHT = 11,     /* RMS norms without their weights */
  OX_PLANT_KEY_HEAD = 12,        /* value head h reads key head h / (VH/KH) */
  OX_PLANT_DELTA_PRED_DECAY = 13, /* prediction from the undecayed state */
  OX_PLANT_SELECT_TIE_HIGH = 14,  /* equal router logits ranked toward the higher index */
  OX_PLANT_SELECT_ASCENDING = 15, /* the K smallest router logits selected */
  OX_PLANT_PROB_UNNORMALISED = 16,/* routing weights not divided by the top-k sum */
  OX_PLANT_SOFTMAX_ALL = 17,      /* routing softmax over all experts, not the top k */
  OX_PLANT_SHARED_GATE = 18,      /* shared expert without its sigmoid gate */
  OX_PLANT_ARGMAX_LAST = 19       /* argmax ties resolved to the last index */
};
void ox_set_plant(int which);

/* Kernel-level entry points for the known-answer tests. */
void ox_project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols, int width,
                uint16_t* out);
void ox_residual_project(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols,
                         const uint16_t* residual, uint16_t* out);
void ox_swiglu_project(const uint16_t* x, const uint16_t* wg, const uint16_t* wu, int64_t rows,
                       int64_t cols, uint16_t* out);
void ox_moe_gate_rows(const uint16_t* x, const uint16_t* gate, const uint16_t* up,
                      const uint16_t* sgate, const uint16_t* sup, const int64_t* ids,
                      const float* probs, float shared_logit, int64_t H, int64_t K, int64_t I,
                      int64_t SI, uint16_t* active);
void ox_moe_down_rows(const uint16_t* active, const uint16_t* down, const uint16_t* sdown,
                      const int64_t* ids, const uint16_t* residual, int64_t H, int64_t K,
                      int64_t I, int64_t SI, uint16_t* out);
void ox_moe_route(const uint16_t* x, const float* router, const float* shared_router, int64_t H,
                  int64_t E, int64_t K, float* logits, int64_t* ids, float* probs);

/* One restated function each, on explicit buffers (per-function pins). */
void ox_k_normalize(const uint16_t* x, const float* w, int64_t cols, int64_t rows, float eps,
                    uint16_t* out);
void ox_k_prepare_heads(const ox_model* m, int64_t position, const uint16_t* in, const float* w,
                        int64_t heads, uint16_t* out);
void ox_k_rope(const ox_model* m, int64_t position, const uint16_t* in, int64_t heads, uint16_t* out);
void ox_k_conv(const ox_model* m, uint16_t* history, int64_t position, const float* weight,
               const uint16_t* qkv, uint16_t* out);
void ox_k_l2(const uint16_t* in, int heads, int dim, uint16_t* out);
void ox_k_delta(const ox_model* m, const uint16_t* conv, const uint16_t* q, const uint16_t* k,
                const uint16_t* alpha, const uint16_t* beta, const float* dt, const float* a,
                uint16_t* state16, float* state32, uint16_t* out);
void ox_k_gated_norm(const ox_model* m, const uint16_t* core, const uint16_t* z, const float* w,
                     uint16_t* out);
void ox_k_attention(const ox_model* m, int online, const uint16_t* q, const uint16_t* kv, int64_t keys,
                    const uint16_t* qg, int64_t split_keys, uint16_t* out);
void ox_k_select(const float* logits, int64_t E, int64_t K, int64_t* ids, float* probs);
uint64_t ox_k_argmax(const uint16_t* logits, int64_t vocab);

#ifdef __cplusplus
}
#endif
#endif
