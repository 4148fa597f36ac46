/*
 * cq35 — MI355X-native Qwen3.5/3.6 token loop behind a plain C ABI.
 *
 * The entry points replace the compiled catena artifact's session ABI that
 * hellas-ai/catena-models' Rust runtime binds (src/model.rs):
 *
 *   qwen3.init(capacity) -> state          src/model.rs:248-258,
 *                                          src/catena/state_init_moe.hex:2-13,
 *                                          src/catena/state_init_hybrid.hex:2-7
 *   qwen3(tokens, state, capacity, start,  src/model.rs:260-328,
 *         weights...) -> state, logits,    src/qwen/qwen35.rs:1466-1650
 *         token
 *   qwen3.copy-buffer(-16)(buffer, n)      src/model.rs:209-246,
 *                                          src/catena/session_copy.hex:131-135
 *   weights placed once in device memory   src/checkpoint.rs:197-231, 822-880
 *   weight ABI order                       src/spec.rs:443-712 (weight_specs)
 *
 * Conventions: every call returns 0 on success or a negative CQ35_E* code;
 * cq35_last_error() describes the last failure of the calling thread. No
 * signature carries framework types: only plain pointers, sizes and scalars.
 * One caller per session at a time; distinct sessions may be used from
 * distinct threads.
 */
#ifndef CQ35_H
#define CQ35_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CQ35_ABI_VERSION 3  /* 3: cq35_session_set_matrix_decode; 2: cq35_step_batch logits */

enum {
  CQ35_OK = 0,
  CQ35_EINVAL = -1,        /* malformed argument or configuration */
  CQ35_ERANGE = -2,        /* token id / position / capacity out of range */
  CQ35_EDEVICE = -3,       /* HIP runtime failure */
  CQ35_EUNSUPPORTED = -4,  /* path not provided by this build */
  CQ35_EPOISONED = -5      /* session state unusable after a failed step */
};

/* The fields of ModelConfig (src/spec.rs:33-62) the token loop reads.
 * moe != 0 selects ModelArchitecture::Qwen35Moe. */
typedef struct cq35_config {
  int32_t moe;
  int32_t vocab;
  int32_t hidden;
  int32_t intermediate;      /* dense FFN width, or per-expert width (MoE) */
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
  int32_t key_heads;         /* linear_group_count */
  int32_t key_dim;           /* linear_state_size */
  int32_t value_heads;       /* linear_time_step_rank */
  int32_t value_dim;         /* linear_inner_size / linear_time_step_rank */
  int32_t tied;              /* output_weight_tied */
} cq35_config;

enum { CQ35_BF16 = 0, CQ35_F32 = 1 };

typedef struct cq35_tensor_info {
  int32_t dtype;      /* CQ35_BF16 or CQ35_F32 */
  int64_t rows;       /* leading dimensions folded: [E,I,H] -> rows=E*I, cols=H */
  int64_t cols;
  int64_t bytes;
} cq35_tensor_info;

typedef struct cq35_model cq35_model;
typedef struct cq35_session cq35_session;

const char* cq35_last_error(void);
int cq35_abi_version(void);

/* ModelConfig::validate (src/spec.rs:185-275) plus the limits of this build. */
int cq35_config_validate(const cq35_config* cfg);

/* weight_specs (src/spec.rs:443-712): tensor count and per-tensor shape. */
int cq35_weight_count(const cq35_config* cfg, int64_t* count);
int cq35_weight_info(const cq35_config* cfg, int64_t index, cq35_tensor_info* info);

/* Place the weights in device memory once (replacing the reference's
 * hipHostRegister zero-copy mapping, src/checkpoint.rs:916-986).
 * weights[i] points at tensor i in weight_specs order; on_device != 0 means
 * the pointers are already device allocations that the caller keeps alive
 * for the model's lifetime (they are borrowed, not copied). */
int cq35_model_create(const cq35_config* cfg, const void* const* weights, int on_device,
                      cq35_model** out);

/* Same, with weights produced on the device by the library's counter-based
 * synthetic generator: per tensor t and element i, SplitMix64 finaliser of
 * mix64(seed ^ mix64(t + 1)) + i * 0x9E3779B97F4A7C15, Irwin-Hall(4)
 * normals; BF16 matrices ~N(0, 0.02), norms 1 + N(0, 0.02), dt 1,
 * A = -(1 + 15u), conv N(0, 0.3), router N(0, 0.04), shared gate N(0, 0.02).
 * No reference counterpart: for benchmarks and parity tests without a
 * checkpoint. */
int cq35_model_create_synthetic(const cq35_config* cfg, uint64_t seed, cq35_model** out);

/* GGUF checkpoints (src/checkpoint.rs): `path` is one version-3 file, any
 * member of a standard shard set (<prefix>-NNNNN-of-MMMMM.gguf; every shard
 * is read) or a directory of .gguf files.
 * cq35_gguf_config: read_gguf_model_config (checkpoint.rs:376-404, 422-639)
 *   for the qwen35 / qwen35moe architectures (others: CQ35_EUNSUPPORTED);
 *   the output head is tied unless an output.weight tensor exists.
 * cq35_gguf_validate: validate_gguf_tensors (checkpoint.rs:406-414, 659-733,
 *   766-820): the tensor inventory equals weight_specs' GGUF names (tensors
 *   of next-token layers aside), each with its shape and dtype, inside its
 *   file, none overlapping. cfg, when given, must equal the metadata's.
 * cq35_model_load_gguf: Model::load_gguf (model.rs:43, 81-153): the above,
 *   then every tensor copied into HBM once (cq35_model_create).
 * cq35_gguf_tensor_name: the GGUF name of weight_specs entry `index`. */
int cq35_gguf_config(const char* path, cq35_config* out);
int cq35_gguf_validate(const char* path, const cq35_config* cfg);
int cq35_model_load_gguf(const char* path, cq35_model** out);
int cq35_gguf_tensor_name(const cq35_config* cfg, int64_t index, char* buf, int64_t len);
int cq35_model_free(cq35_model* model);
int cq35_model_config(const cq35_model* model, cq35_config* out);
/* Device bytes held by the model's weights. */
int cq35_model_weight_bytes(const cq35_model* model, int64_t* bytes);
/* Copy tensor `index` back to host memory (for checks). */
int cq35_model_read_weight(const cq35_model* model, int64_t index, void* dst, int64_t bytes);

/* qwen3.init: zero-initialised opaque state for `capacity` positions. */
int cq35_session_init(cq35_model* model, int64_t capacity, cq35_session** out);
int cq35_session_free(cq35_session* session);

/* qwen3: process tokens[0..n) at positions start..start+n (n == 1 is the
 * decode step), write the greedy next token and, when logits != NULL, the
 * final position's BF16 logits (vocab entries) to host memory.
 * `capacity` must equal the session's. A failure after work was enqueued
 * poisons the session (the reference drops its state on a failed exec,
 * src/model.rs:711-730). */
int cq35_step(cq35_session* session, const uint64_t* tokens, int64_t n, int64_t start,
              int64_t capacity, uint64_t* next_token, uint16_t* logits);

/* One decode step (one token each) for several independent sessions:
 * tokens[i] at position starts[i] of sessions[i], next token into
 * next_tokens[i] and, when logits != NULL, session i's BF16 logits into
 * logits[i * vocab ..]. Dense sessions of one model and capacity take one
 * weight-shared step (each layer's weights read once for all of them); each
 * session's result is then identical to its own cq35_step, unless every
 * session of the batch selects matrix-core decode
 * (cq35_session_set_matrix_decode), in which case the products run on MFMA
 * (hardware accumulation order: tolerance-level, like the matrix-core
 * prefill). Other sessions on the per-kernel path are launched back to back
 * on their own streams and then completed, so their kernels overlap on the
 * device; sessions on the persistent path step one at a time (each launch
 * needs every CU). All checks precede any work. If a step fails after work
 * was enqueued, every session of the batch is poisoned (some may have
 * advanced a position; none reports a token). No reference counterpart: the
 * reference steps sessions one after another (src/server/engine.rs:143-207);
 * this is the entry point for batch-16 serving. */
int cq35_step_batch(cq35_session* const* sessions, const uint64_t* tokens, const int64_t* starts,
                    int64_t count, uint64_t* next_tokens, uint16_t* logits);

/* A decode step (one token) that allocates nothing, for callers that cannot
 * allocate device memory: tight serving loops and harnesses that forbid
 * hipMalloc. No counterpart in the reference.
 * `state` is caller-owned device memory holding the BF16 session state of
 * `capacity` positions in the reference layout (cq35_session_state_bytes
 * with which = 0, e.g. copied from cq35_session_export_state); it is updated
 * in place exactly as cq35_step updates a session (same per-kernel decode
 * sequence, same results). `stream` is a hipStream_t (NULL: the default
 * stream); the call waits for it before returning the greedy token and, when
 * logits != NULL, the BF16 logits to host memory. Every other buffer comes
 * from one static device array of 16 MiB per device (held until the process
 * ends), which bounds the capacity: about 80K positions at the 35B-A3B shape;
 * larger capacities are rejected with CQ35_ERANGE before any work. Calls on
 * one device share that array: each holds a per-device lock from its first
 * launch until its stream has drained, so calls from several threads or
 * streams of one device run one after another. The call synchronises its
 * stream before returning, so it cannot run under HIP graph capture.
 * Decode attention splits above CQ35_SPLIT_KEYS_DEFAULT cached keys, as a
 * new session's does (there is no per-call threshold; at the capacities
 * this call accepts the split applies above 8192 positions). */
int cq35_step_static(const cq35_model* model, uint16_t* state, int64_t capacity, uint64_t token,
                     int64_t start, void* stream, uint64_t* next_token, uint16_t* logits);

/* qwen3.copy-buffer (session_copy.hex:131-135; src/model.rs:209-246): an
 * independent bitwise copy of a session's state and options. */
int cq35_session_copy(const cq35_session* src, cq35_session** out);

/* Canonical state for parity checks, in the reference layout
 * (state_layout.hex, decoder.hex:16-23, qwen35.hex:2-16):
 *   which = 0: BF16 cache [KV: layer, K|V, capacity, kv_heads*head_dim]
 *              [per layer: conv history 3*QKV, recurrent VH*VD*KD]
 *   which = 1: F32 DeltaNet shadow [layer, VH*VD*KD]
 *   which = 2: (MoE only, export only) int32 [layer, top_k]: the expert ids
 *              in rank order that the last call's final token selected at
 *              each layer (the reference keeps the current layer's ids in
 *              its workspace, state_layout.hex:53-87, written by
 *              qwen35_moe.hex:86-252)
 * `bytes` must equal cq35_session_state_bytes(session, which). */
int cq35_session_state_bytes(const cq35_session* session, int which, int64_t* bytes);
int cq35_session_export_state(const cq35_session* session, int which, void* dst, int64_t bytes);
int cq35_session_import_state(cq35_session* session, int which, const void* src, int64_t bytes);

/* Measurement hooks (no reference counterpart): time every launch of one
 * kernel class with start/stop events stamped by its dispatch packet on the
 * session stream (class ids: see cq35_kernel_class_name); -1 disables.
 * Results accumulate until read. Decode-step graph replay is suspended while
 * timing is on. */
int cq35_session_time_kernel(cq35_session* session, int kernel_class);
int cq35_session_kernel_time(cq35_session* session, double* total_ms, int64_t* launches);
const char* cq35_kernel_class_name(int kernel_class);
int cq35_kernel_class_count(void);
/* Phase stamps of the last persistent decode step, in a library built with
 * -DCQ35_PHASE_TRACE (otherwise CQ35_EUNSUPPORTED): `*slots` stamps per
 * block (s_memrealtime, 100 MHz) for each of the `*blocks` blocks of the
 * step; with dst != NULL, count must be blocks x slots. Slot meanings:
 * mega.h, phase trace. No reference counterpart (measurement only). */
int cq35_session_phase_trace(const cq35_session* session, uint64_t* dst, int64_t count, int64_t* slots,
                             int64_t* blocks);
/* Disable (0) or enable (1, default) hipGraph replay of the decode step. */
int cq35_session_set_graph(cq35_session* session, int enabled);

/* Decode steps (n == 1) of MoE models run as one persistent launch per token
 * by default, where the shape and capacity fit its limits; 0 selects the
 * per-kernel launch sequence, 1 the persistent kernel (CQ35_EUNSUPPORTED
 * when the session's shape is outside it). Same arithmetic either way. No
 * reference counterpart (the reference launches ~1,316 kernels per token). */
int cq35_session_set_persistent(cq35_session* session, int enabled);
int cq35_session_persistent(const cq35_session* session, int* enabled);

/* Split-K decode attention for long contexts. Over more than `keys` cached
 * keys (default CQ35_SPLIT_KEYS_DEFAULT; 0: never) the T tiles (8 keys) of
 * each query head's online softmax form at most 128 ranges of ceil(T / 128)
 * tiles, each the reference's recurrence over its own tiles from scratch,
 * merged in ascending range order (M = max m_r, w_r = exp(m_r - M),
 * den = 0 + d_0 w_0 + d_1 w_1 + ..., likewise each channel). The reference
 * runs one sequential chain over all tiles (qwen35_online.hex:272-331); the
 * split changes rounding only (tolerance-level), and at or below the
 * threshold the result is the reference's bit for bit. Both decode paths use
 * the same ranges, which depend on the key count alone. */
#define CQ35_SPLIT_KEYS_DEFAULT 8192
int cq35_session_set_attention_split(cq35_session* session, int64_t keys);
int cq35_session_attention_split(const cq35_session* session, int64_t* keys);

/* Matrix-core prefill: components of multi-token calls run on MFMA, whose
 * F32 accumulation order is the hardware's, so results match the exact path
 * to accumulation rounding rather than bit for bit. Replaces the reference's
 * InferenceOptions::wmma_prefill with CATENA_WMMA_COMPONENTS (catena.rs:12-26,
 * qwen35.rs:467-541; default off in its library API, as here). Bit 0: the
 * dense projections (attention, DeltaNet and output projections, dense FFN);
 * bit 1: the MoE expert projections (grouped routed experts and the shared
 * expert); bit 2: the full-attention layers' attention over the prompt rows
 * (scores and context on MFMA with the reference's BF16 score, probability
 * and context rounding, qwen35_wmma_attention.hex; head_dim 64, 128 or 256,
 * other head dims keep the exact kernels). 0 keeps the exact SIMT path. A
 * session whose components are set at its first multi-token call runs
 * multi-token calls in chunks of 1024 tokens (otherwise 256; the chunk
 * changes no result). Decode steps (cq35_step with n == 1, and
 * cq35_step_batch) are unaffected, as the reference's option affects prefill
 * only. */
#define CQ35_MATRIX_PROJECTIONS 1
#define CQ35_MATRIX_EXPERTS 2
#define CQ35_MATRIX_ATTENTION 4
int cq35_session_set_matrix_prefill(cq35_session* session, int components);
int cq35_session_matrix_prefill(const cq35_session* session, int* components);

/* Matrix-core batched decode (no reference counterpart): 1 lets the
 * weight-shared step of cq35_step_batch run its products on MFMA (hardware
 * accumulation order, tolerance-level) for a batch in which EVERY session has
 * this option set; a batch with any session at 0 (the default) takes the
 * exact products, so each session's tokens are then identical to its own
 * cq35_step. Single-session steps are unaffected. Copied by
 * cq35_session_copy. */
int cq35_session_set_matrix_decode(cq35_session* session, int enabled);
int cq35_session_matrix_decode(const cq35_session* session, int* enabled);

/* Host-side builds of the device numerics (same source), for CPU checks. */
float cq35_numeric_exp(float x);
float cq35_numeric_sqrt(float x);
float cq35_numeric_softplus(float x);
void cq35_numeric_sincos(float angle, float* sine, float* cosine);
/* Device evaluation of the same numerics over an array (op 0 exp, 1 silu,
 * 2 sigmoid, 3 softplus, 4 sqrt, 5 sin, 6 cos, 7 the F32 -> BF16 rounding
 * widened back to F32); host in/out arrays. */
int cq35_device_numeric(int op, const float* input, float* output, int64_t count);
/* Device split-pair GEMV with tree width W (32, 64 or 256) over a row-major
 * BF16 matrix: out[r] = bf16(tree_W(x . w_r)). Host arrays. */
int cq35_device_gemv(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols,
                     int width, uint16_t* out);
/* Device matrix-core product of the prefill projections over host arrays,
 * x [n][cols], w and w2 [rows][cols], res [n][rows], cols a multiple of 16:
 * out[t][r] = epilogue(sum_k x[t][k] w[r][k]) in the MFMA accumulation order,
 * mode 0 bf16(sum), 1 bf16(sum) (+) res, 2 bf16(silu(bf16 sum)) (x)
 * bf16(sum over w2). kernel 0: direct fragment loads; 1: the LDS-staged
 * tiles the prefill runs (the same order, so the same bits). */
int cq35_device_matrix_gemm(const uint16_t* x, const uint16_t* w, const uint16_t* w2,
                            const uint16_t* res, int64_t n, int64_t rows, int64_t cols, int mode,
                            int kernel, uint16_t* out);
/* Device matrix-core attention of the prompt path (CQ35_MATRIX_ATTENTION's
 * kernel) over host arrays: n query rows at positions start .. start + n - 1
 * against keys 0 .. start + n - 1. q and gate [n][heads][head_dim] (q
 * normalised and rotated), k and v [start + n][kv_heads][head_dim], out
 * [n][heads][head_dim] = bf16(bf16(sum_j p_j v_j) * sigmoid(gate)) with
 * p_j = bf16(exp(s_j - max) / den) and s_j = bf16(q . k_j / sqrt(head_dim))
 * over the keys j at or before the row's position, the products on MFMA.
 * head_dim 64, 128 or 256; heads a multiple of kv_heads. */
int cq35_device_matrix_attention(const uint16_t* q, const uint16_t* gate, const uint16_t* k,
                                 const uint16_t* v, int64_t n, int64_t start, int heads, int kv_heads,
                                 int head_dim, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
