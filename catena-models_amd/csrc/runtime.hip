// Host side of the cq35 C ABI: configuration and weight ABI, device weight
// placement, sessions with the reference's opaque state layout, and the
// per-token launch sequence (captured once into a hipGraph for decode).
//
// Reference call path replaced: src/model.rs:260-328 (Model::cached_outputs
// -> Artifact::exec_values("qwen3")), src/qwen/qwen35.rs:1374-1650 (the
// generated token fold), src/model.rs:248-258 (qwen3.init).
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>
#include <string>
#include <vector>

#include "../../include/cq35.h"
#include "attention.h"
#include "layers.h"
#include "mega.h"
#include "dense_step.h"
#include "prefill.h"
#include "mfma.h"
#include "gguf.h"
#include "batch.h"
#include "batch_moe.h"

using namespace cq35;

// ----------------------------------------------------------------- errors

static thread_local std::string g_error;

static int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

#define HIP_TRY(expr)                                                                     \
  do {                                                                                    \
    hipError_t e_ = (expr);                                                               \
    if (e_ != hipSuccess)                                                                 \
      return fail(CQ35_EDEVICE, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_),     \
                  __FILE__, __LINE__);                                                    \
  } while (0)

extern "C" const char* cq35_last_error(void) { return g_error.c_str(); }
extern "C" int cq35_abi_version(void) { return CQ35_ABI_VERSION; }

// ----------------------------------------------------------- configuration

namespace {

struct Dims {
  int64_t H, V, L, Q, KVH, HD, R, KS, VS, QKV, REC, CONV, LIN, KVS, QS, KV_STRIDE, E, K, I, SI;
  int pad_h, pad_hd;
};

int64_t next_pow2(int64_t v) {
  int64_t p = 1;
  while (p < v) p <<= 1;
  return p;
}

Dims dims_of(const cq35_config& c) {
  Dims d{};
  d.H = c.hidden; d.V = c.vocab; d.L = c.layers; d.Q = c.q_heads; d.KVH = c.kv_heads;
  d.HD = c.head_dim; d.R = c.rope_dim;
  d.KS = (int64_t)c.key_heads * c.key_dim;
  d.VS = (int64_t)c.value_heads * c.value_dim;
  d.QKV = 2 * d.KS + d.VS;
  d.REC = d.VS * c.key_dim;
  d.CONV = 3 * d.QKV;
  d.LIN = d.CONV + d.REC;
  d.KVS = d.KVH * d.HD;
  d.QS = d.Q * d.HD;
  d.KV_STRIDE = d.L * 2 * d.KVS;
  d.E = c.experts; d.K = c.top_k; d.I = c.intermediate; d.SI = c.shared_intermediate;
  d.pad_h = (int)next_pow2(d.H);
  d.pad_hd = (int)next_pow2(d.HD);
  return d;
}

bool is_full(const cq35_config& c, int64_t l) { return ((l + 1) % c.full_interval) == 0; }
int layer_tensors(const cq35_config& c, int64_t l) {
  return is_full(c, l) ? (c.moe ? 16 : 11) : (c.moe ? 19 : 14);
}

// Kinds drive the synthetic generator (shared specification with the CPU
// restatement): BF16 matrices ~N(0, 0.02); norm weights 1 + N(0, 0.02);
// dt bias 1; A = -(1 + 15u); conv taps N(0, 0.3); router N(0, 0.04);
// shared-expert gate row N(0, 0.02).
struct TensorDesc {
  int32_t dtype;
  int64_t rows, cols;
  int kind;
};

int64_t weight_count(const cq35_config& c) {
  int64_t n = 1;
  for (int64_t l = 0; l < c.layers; ++l) n += layer_tensors(c, l);
  return n + 2;
}

// src/spec.rs:443-712, in order.
bool describe(const cq35_config& c, int64_t index, TensorDesc* t) {
  const Dims d = dims_of(c);
  const int64_t total = weight_count(c);
  auto set = [&](int32_t dt, int64_t r, int64_t co, int kind) {
    *t = TensorDesc{dt, r, co, kind};
    return true;
  };
  if (index < 0 || index >= total) return false;
  if (index == 0) return set(CQ35_BF16, d.V, d.H, kEmbed);
  if (index == total - 2) return set(CQ35_F32, d.H, 1, kNorm);
  if (index == total - 1) return set(CQ35_BF16, d.V, d.H, kEmbed);
  int64_t base = 1;
  for (int64_t l = 0; l < c.layers; ++l) {
    const int n = layer_tensors(c, l);
    if (index < base + n) {
      const int s = (int)(index - base);
      if (s == 0) return set(CQ35_F32, d.H, 1, kNorm);
      int ffn;
      if (is_full(c, l)) {
        switch (s) {
          case 1: return set(CQ35_BF16, 2 * d.QS, d.H, kMatrix);
          case 2: return set(CQ35_BF16, d.KVS, d.H, kMatrix);
          case 3: return set(CQ35_BF16, d.KVS, d.H, kMatrix);
          case 4: return set(CQ35_BF16, d.H, d.QS, kMatrix);
          case 5: return set(CQ35_F32, d.HD, 1, kNorm);
          case 6: return set(CQ35_F32, d.HD, 1, kNorm);
          case 7: return set(CQ35_F32, d.H, 1, kNorm);
          default: break;
        }
        ffn = s - 8;
      } else {
        switch (s) {
          case 1: return set(CQ35_BF16, d.QKV, d.H, kMatrix);
          case 2: return set(CQ35_BF16, d.VS, d.H, kMatrix);
          case 3: return set(CQ35_BF16, c.value_heads, d.H, kMatrix);
          case 4: return set(CQ35_BF16, c.value_heads, d.H, kMatrix);
          case 5: return set(CQ35_F32, c.value_heads, 1, kDt);
          case 6: return set(CQ35_F32, c.value_heads, 1, kA);
          case 7: return set(CQ35_F32, c.value_dim, 1, kNorm);
          case 8: return set(CQ35_BF16, d.H, d.VS, kMatrix);
          case 9: return set(CQ35_F32, d.QKV, 4, kConv);
          case 10: return set(CQ35_F32, d.H, 1, kNorm);
          default: break;
        }
        ffn = s - 11;
      }
      if (!c.moe) {
        switch (ffn) {
          case 0: return set(CQ35_BF16, d.I, d.H, kMatrix);
          case 1: return set(CQ35_BF16, d.I, d.H, kMatrix);
          case 2: return set(CQ35_BF16, d.H, d.I, kMatrix);
          default: return false;
        }
      }
      switch (ffn) {
        case 0: return set(CQ35_F32, d.E, d.H, kRouter);
        case 1: return set(CQ35_BF16, d.E * d.I, d.H, kMatrix);
        case 2: return set(CQ35_BF16, d.E * d.I, d.H, kMatrix);
        case 3: return set(CQ35_BF16, d.E * d.H, d.I, kMatrix);
        case 4: return set(CQ35_F32, 1, d.H, kSharedGate);
        case 5: return set(CQ35_BF16, d.SI, d.H, kMatrix);
        case 6: return set(CQ35_BF16, d.SI, d.H, kMatrix);
        case 7: return set(CQ35_BF16, d.H, d.SI, kMatrix);
        default: return false;
      }
    }
    base += n;
  }
  return false;
}

// GGUF name, reference shape (outermost first) and dtype of tensor `index`
// in weight_specs order (src/spec.rs:443-712: gguf_name and shape).
bool gguf_spec(const cq35_config& c, int64_t index, std::string* name, std::vector<uint64_t>* dims,
               int32_t* dtype) {
  TensorDesc t;
  if (!describe(c, index, &t)) return false;
  *dtype = t.dtype;
  const Dims d = dims_of(c);
  const int64_t total = weight_count(c);
  auto set = [&](const std::string& n, std::vector<uint64_t> sh) {
    *name = n;
    *dims = std::move(sh);
    return true;
  };
  const uint64_t H = d.H, V = d.V;
  if (index == 0) return set("token_embd.weight", {V, H});
  if (index == total - 2) return set("output_norm.weight", {H});
  if (index == total - 1) return set(c.tied ? "token_embd.weight" : "output.weight", {V, H});
  int64_t base = 1;
  for (int64_t l = 0; l < c.layers; ++l) {
    const int n = layer_tensors(c, l);
    if (index < base + n) {
      const int s = (int)(index - base);
      const std::string b = "blk." + std::to_string(l) + ".";
      if (s == 0) return set(b + "attn_norm.weight", {H});
      int ffn;
      if (is_full(c, l)) {
        switch (s) {
          case 1: return set(b + "attn_q.weight", {(uint64_t)(2 * d.QS), H});
          case 2: return set(b + "attn_k.weight", {(uint64_t)d.KVS, H});
          case 3: return set(b + "attn_v.weight", {(uint64_t)d.KVS, H});
          case 4: return set(b + "attn_output.weight", {H, (uint64_t)d.QS});
          case 5: return set(b + "attn_q_norm.weight", {(uint64_t)d.HD});
          case 6: return set(b + "attn_k_norm.weight", {(uint64_t)d.HD});
          case 7: return set(b + "post_attention_norm.weight", {H});
          default: break;
        }
        ffn = s - 8;
      } else {
        const uint64_t VH = (uint64_t)c.value_heads;
        switch (s) {
          case 1: return set(b + "attn_qkv.weight", {(uint64_t)d.QKV, H});
          case 2: return set(b + "attn_gate.weight", {(uint64_t)d.VS, H});
          case 3: return set(b + "ssm_alpha.weight", {VH, H});
          case 4: return set(b + "ssm_beta.weight", {VH, H});
          case 5: return set(b + "ssm_dt.bias", {VH});
          case 6: return set(b + "ssm_a", {VH});
          case 7: return set(b + "ssm_norm.weight", {(uint64_t)c.value_dim});
          case 8: return set(b + "ssm_out.weight", {H, (uint64_t)d.VS});
          case 9: return set(b + "ssm_conv1d.weight", {(uint64_t)d.QKV, 4});
          case 10: return set(b + "post_attention_norm.weight", {H});
          default: break;
        }
        ffn = s - 11;
      }
      const uint64_t I = d.I, E = d.E, SI = d.SI;
      if (!c.moe) {
        switch (ffn) {
          case 0: return set(b + "ffn_gate.weight", {I, H});
          case 1: return set(b + "ffn_up.weight", {I, H});
          case 2: return set(b + "ffn_down.weight", {H, I});
          default: return false;
        }
      }
      switch (ffn) {
        case 0: return set(b + "ffn_gate_inp.weight", {E, H});
        case 1: return set(b + "ffn_gate_exps.weight", {E, I, H});
        case 2: return set(b + "ffn_up_exps.weight", {E, I, H});
        case 3: return set(b + "ffn_down_exps.weight", {E, H, I});
        case 4: return set(b + "ffn_gate_inp_shexp.weight", {1, H});
        case 5: return set(b + "ffn_gate_shexp.weight", {SI, H});
        case 6: return set(b + "ffn_up_shexp.weight", {SI, H});
        case 7: return set(b + "ffn_down_shexp.weight", {H, SI});
        default: return false;
      }
    }
    base += n;
  }
  return false;
}

int64_t tensor_bytes(const TensorDesc& t) { return t.rows * t.cols * (t.dtype == CQ35_BF16 ? 2 : 4); }

int64_t cache_elements(const cq35_config& c, int64_t capacity) {
  // src/spec.rs:321-362 = state_layout.hex:26-27
  const Dims d = dims_of(c);
  return capacity * d.KV_STRIDE + d.L * d.LIN;
}

}  // namespace

extern "C" int cq35_config_validate(const cq35_config* cfg) {
  if (!cfg) return fail(CQ35_EINVAL, "null configuration");
  const cq35_config& c = *cfg;
  // ModelConfig::validate (src/spec.rs:185-275).
  if (c.vocab <= 0 || c.hidden <= 0 || c.intermediate <= 0 || c.layers <= 0 || c.q_heads <= 0 ||
      c.kv_heads <= 0 || c.head_dim <= 0)
    return fail(CQ35_EINVAL, "model dimensions must be non-zero");
  if (c.q_heads % c.kv_heads != 0)
    return fail(CQ35_EINVAL, "attention head count must be divisible by KV head count");
  if (c.moe) {
    if (c.experts <= 0 || c.top_k <= 0) return fail(CQ35_EINVAL, "expert counts must be non-zero");
    if (c.top_k > c.experts) return fail(CQ35_EINVAL, "experts used exceeds expert count");
    if (c.shared_intermediate <= 0) return fail(CQ35_EINVAL, "missing shared expert size");
  } else if (c.experts != 0 || c.top_k != 0) {
    return fail(CQ35_EINVAL, "dense model metadata must not define routed experts");
  }
  if (c.rope_dim <= 0 || c.rope_dim > c.head_dim)
    return fail(CQ35_EINVAL, "rotary dimension must be within the attention head");
  if (c.full_interval <= 0 || c.key_heads <= 0 || c.key_dim <= 0 || c.value_heads <= 0 ||
      c.value_dim <= 0)
    return fail(CQ35_EINVAL, "hybrid layer metadata must be non-zero");
  bool has_full = false, has_linear = false;
  for (int l = 0; l < c.layers; ++l) (is_full(c, l) ? has_full : has_linear) = true;
  if (!has_full || !has_linear)
    return fail(CQ35_EINVAL, "Qwen3.5 requires both full and linear layers");
  // Limits of this build's kernels.
  if (c.hidden % 8 || c.intermediate % 8 || (c.moe && c.shared_intermediate % 8) ||
      (c.q_heads * c.head_dim) % 8 || (c.value_heads * c.value_dim) % 8)
    return fail(CQ35_EINVAL, "widths must be multiples of 8 elements (128-bit GEMV loads)");
  if (c.head_dim > 256 || c.key_dim > 256 || c.value_dim > 256 || c.key_dim % 32 || c.head_dim % 32)
    return fail(CQ35_EINVAL, "head_dim/key_dim multiples of 32 up to 256, value_dim <= 256");
  if ((c.q_heads / c.kv_heads) * c.head_dim > 16 * 256)
    return fail(CQ35_EINVAL, "at most 16 query heads of 256 channels per KV head");
  if (c.rope_dim % 2) return fail(CQ35_EINVAL, "rotary dimension must be even");
  if (c.moe && (c.experts > 4096 || c.top_k > 64))
    return fail(CQ35_EINVAL, "at most 4096 experts and top-k 64");
  if (c.value_dim % 8) return fail(CQ35_EINVAL, "value head width must be a multiple of 8");
  if (c.hidden > 16384) return fail(CQ35_EINVAL, "hidden width above 16384");
  if ((int64_t)c.q_heads * c.head_dim > 32768 || (int64_t)c.value_heads * c.value_dim > 32768 ||
      (!c.moe && c.intermediate > 32768))
    return fail(CQ35_EINVAL, "residual projection inputs above 32768 values");
  if (c.moe && (int64_t)c.top_k * c.intermediate + c.shared_intermediate > 12288)
    return fail(CQ35_EINVAL, "top_k * intermediate + shared_intermediate above 12288");
  return CQ35_OK;
}

extern "C" int cq35_weight_count(const cq35_config* cfg, int64_t* count) {
  int rc = cq35_config_validate(cfg);
  if (rc) return rc;
  if (!count) return fail(CQ35_EINVAL, "null output");
  *count = weight_count(*cfg);
  return CQ35_OK;
}

extern "C" int cq35_weight_info(const cq35_config* cfg, int64_t index, cq35_tensor_info* info) {
  int rc = cq35_config_validate(cfg);
  if (rc) return rc;
  TensorDesc t;
  if (!info || !describe(*cfg, index, &t)) return fail(CQ35_EINVAL, "bad weight index %lld", (long long)index);
  info->dtype = t.dtype;
  info->rows = t.rows;
  info->cols = t.cols;
  info->bytes = tensor_bytes(t);
  return CQ35_OK;
}

// ------------------------------------------------------------------ model

namespace {
struct BatchWorkspace;
void destroy_batch(BatchWorkspace* b);
}  // namespace

struct cq35_model {
  cq35_config cfg;
  Dims d;
  int device = 0;
  std::vector<void*> w;       // device pointers in weight ABI order
  std::vector<void*> owned;   // allocations to free
  float* freq = nullptr;      // F32 theta^(-2i/R) (src/catena.rs:185-232)
  int64_t weight_bytes = 0;
  std::mutex batch_lock;      // one weight-shared batched step at a time
  BatchWorkspace* batch = nullptr;  // its buffers (allocated on first use)
};

namespace {

int finish_model(cq35_model* m) {
  const int half = (int)(m->cfg.rope_dim / 2);
  std::vector<float> f(std::max(half, 1));
  for (int i = 0; i < half; ++i)
    f[i] = powf(m->cfg.theta, -((float)(2 * i) / (float)m->cfg.rope_dim));
  HIP_TRY(hipMalloc(&m->freq, f.size() * sizeof(float)));
  HIP_TRY(hipMemcpy(m->freq, f.data(), f.size() * sizeof(float), hipMemcpyHostToDevice));
  return CQ35_OK;
}

float normal_scale(double sd) { return (float)(sd / std::sqrt(1431655765.0)); }

}  // namespace

extern "C" int cq35_model_free(cq35_model* m) {
  if (!m) return CQ35_OK;
  hipSetDevice(m->device);
  destroy_batch(m->batch);
  for (void* p : m->owned) hipFree(p);
  if (m->freq) hipFree(m->freq);
  delete m;
  return CQ35_OK;
}

extern "C" int cq35_model_create(const cq35_config* cfg, const void* const* weights, int on_device,
                                 cq35_model** out) {
  int rc = cq35_config_validate(cfg);
  if (rc) return rc;
  if (!weights || !out) return fail(CQ35_EINVAL, "null argument");
  cq35_model* m = new (std::nothrow) cq35_model();
  if (!m) return fail(CQ35_EINVAL, "out of host memory");
  m->cfg = *cfg;
  m->d = dims_of(*cfg);
  hipGetDevice(&m->device);
  const int64_t n = weight_count(*cfg);
  m->w.assign(n, nullptr);
  for (int64_t i = 0; i < n; ++i) {
    TensorDesc t;
    describe(*cfg, i, &t);
    if (!weights[i]) { cq35_model_free(m); return fail(CQ35_EINVAL, "weight %lld is null", (long long)i); }
    const int64_t bytes = tensor_bytes(t);
    if (on_device) {
      m->w[i] = const_cast<void*>(weights[i]);
    } else {
      if (i == n - 1 && weights[i] == weights[0]) { m->w[i] = m->w[0]; continue; }  // tied head
      void* p = nullptr;
      hipError_t e = hipMalloc(&p, bytes);
      if (e == hipSuccess) e = hipMemcpy(p, weights[i], bytes, hipMemcpyHostToDevice);
      if (e != hipSuccess) {
        if (p) hipFree(p);
        cq35_model_free(m);
        return fail(CQ35_EDEVICE, "uploading weight %lld: %s", (long long)i, hipGetErrorString(e));
      }
      m->owned.push_back(p);
      m->w[i] = p;
      m->weight_bytes += bytes;
    }
  }
  rc = finish_model(m);
  if (rc) { cq35_model_free(m); return rc; }
  *out = m;
  return CQ35_OK;
}

namespace {

// parse_gguf_model_config (checkpoint.rs:422-639) for qwen35 / qwen35moe,
// with read_gguf_model_config's tied-output and dtype checks (376-404).
int gguf_config_of(const gguf::Checkpoint& ck, cq35_config* out, uint64_t* nextn) {
  if (ck.arch.empty()) return fail(CQ35_EINVAL, "GGUF is missing general.architecture");
  if (ck.arch != "qwen35" && ck.arch != "qwen35moe")
    return fail(CQ35_EUNSUPPORTED, "GGUF architecture \"%s\" is outside this build (qwen35, qwen35moe)",
                ck.arch.c_str());
  const std::string a = ck.arch;
  int rc = CQ35_OK;
  auto get = [&](const char* key, bool required, bool want_float) -> gguf::Scalar {
    auto it = ck.scalars.find(key);
    if (it == ck.scalars.end()) {
      if (required && !rc) rc = fail(CQ35_EINVAL, "GGUF is missing %s.%s", a.c_str(), key);
      return gguf::Scalar{};
    }
    if (!want_float && it->second.is_float && !rc)
      rc = fail(CQ35_EINVAL, "GGUF %s.%s is not an integer", a.c_str(), key);
    return it->second;
  };
  auto has = [&](const char* key) { return ck.scalars.count(key) != 0; };
  auto u = [&](const char* key) { return get(key, true, false).u; };
  auto ou = [&](const char* key, uint64_t dflt) { return has(key) ? get(key, false, false).u : dflt; };
  auto f = [&](const char* key) {
    const gguf::Scalar s = get(key, true, true);
    return s.is_float ? (float)s.f : (float)s.u;
  };
  const bool moe = a == "qwen35moe";
  cq35_config c{};
  c.moe = moe ? 1 : 0;
  const uint64_t hidden = u("embedding_length"), heads = u("attention.head_count");
  const uint64_t blocks = u("block_count"), nn = ou("nextn_predict_layers", 0);
  if (rc) return rc;
  if (nn >= blocks) return fail(CQ35_EINVAL, "GGUF next-token layer count must be smaller than block count");
  if (!has("vocab_size") && !ck.has_tokens)
    return fail(CQ35_EINVAL, "GGUF has neither %s.vocab_size nor tokenizer tokens", a.c_str());
  const uint64_t vocab = has("vocab_size") ? u("vocab_size") : ck.token_count;
  const uint64_t head_dim = has("attention.key_length") ? u("attention.key_length") : (heads ? hidden / heads : 0);
  const uint64_t inter = moe ? u("expert_feed_forward_length") : u("feed_forward_length");
  const uint64_t kv = u("attention.head_count_kv");
  const float eps = f("attention.layer_norm_rms_epsilon"), theta = f("rope.freq_base");
  const uint64_t rope = ou("rope.dimension_count", head_dim);
  const uint64_t rank = u("ssm.time_step_rank"), inner = u("ssm.inner_size");
  const uint64_t groups = u("ssm.group_count"), state = u("ssm.state_size");
  const uint64_t conv = u("ssm.conv_kernel"), interval = u("full_attention_interval");
  if (rc) return rc;
  if (conv != 4) return fail(CQ35_EINVAL, "Qwen3.5 requires four convolution taps (GGUF has %llu)", (unsigned long long)conv);
  if (rank == 0 || inner % rank) return fail(CQ35_EINVAL, "GGUF ssm.inner_size is not a multiple of ssm.time_step_rank");
  auto i32 = [](uint64_t v) { return v > 0x7fffffffull ? (int32_t)-1 : (int32_t)v; };
  c.vocab = i32(vocab);
  c.hidden = i32(hidden);
  c.intermediate = i32(inter);
  c.layers = i32(blocks - nn);
  c.q_heads = i32(heads);
  c.kv_heads = i32(kv);
  c.head_dim = i32(head_dim);
  c.rope_dim = i32(rope);
  c.eps = eps;
  c.theta = theta;
  c.experts = i32(ou("expert_count", 0));
  c.top_k = i32(ou("expert_used_count", 0));
  c.shared_intermediate = i32(ou("expert_shared_feed_forward_length", 0));
  c.full_interval = i32(interval);
  c.key_heads = i32(groups);
  c.key_dim = i32(state);
  c.value_heads = i32(rank);
  c.value_dim = i32(inner / rank);
  c.tied = ck.tensors.count("output.weight") ? 0 : 1;
  for (const auto& kvp : ck.tensors)
    if (kvp.second.type == gguf::kF16)
      return fail(CQ35_EINVAL, "language GGUF weights must be BF16/F32 (%s is F16)", kvp.first.c_str());
  rc = cq35_config_validate(&c);
  if (rc) return rc;
  *out = c;
  if (nextn) *nextn = nn;
  return CQ35_OK;
}

// validate_files + tensor_view (checkpoint.rs:659-820): the inventory equals
// weight_specs' names (next-token layers aside), every tensor has its
// reference shape and dtype and lies inside its file, and no two overlap.
int gguf_check(const gguf::Checkpoint& ck, const cq35_config& c, uint64_t nextn,
               std::vector<const void*>* pointers) {
  const int64_t n = weight_count(c);
  std::set<std::string> expected;
  std::vector<std::string> names(n);
  std::vector<std::vector<uint64_t>> dims(n);
  std::vector<int32_t> dtypes(n);
  for (int64_t i = 0; i < n; ++i) {
    if (!gguf_spec(c, i, &names[i], &dims[i], &dtypes[i]))
      return fail(CQ35_EINVAL, "no weight spec for tensor %lld", (long long)i);
    expected.insert(names[i]);
  }
  auto auxiliary = [&](const std::string& name) {
    if (nextn == 0 || name.compare(0, 4, "blk.") != 0) return false;
    const size_t dot = name.find('.', 4);
    if (dot == std::string::npos) return false;
    const std::string num = name.substr(4, dot - 4);
    if (num.empty() || !std::all_of(num.begin(), num.end(), [](char ch) { return ch >= '0' && ch <= '9'; }))
      return false;
    const uint64_t layer = std::stoull(num);
    return layer >= (uint64_t)c.layers && layer < (uint64_t)c.layers + nextn;
  };
  std::string missing, unexpected;
  int nm = 0, nu = 0;
  for (const auto& e : expected)
    if (!ck.tensors.count(e) && nm++ < 8) missing += (missing.empty() ? "" : ", ") + e;
  for (const auto& kvp : ck.tensors)
    if (!expected.count(kvp.first) && !auxiliary(kvp.first) && nu++ < 8)
      unexpected += (unexpected.empty() ? "" : ", ") + kvp.first;
  if (nm || nu)
    return fail(CQ35_EINVAL, "GGUF tensor inventory mismatch: %d missing (%s), %d unexpected (%s)", nm,
                missing.c_str(), nu, unexpected.c_str());
  std::vector<std::vector<std::pair<uint64_t, uint64_t>>> ranges(ck.files.size());
  pointers->assign(n, nullptr);
  for (int64_t i = 0; i < n; ++i) {
    const gguf::Tensor& t = ck.tensors.at(names[i]);
    if (t.dims != dims[i]) {
      std::string got, want;
      for (uint64_t v : t.dims) got += (got.empty() ? "" : ",") + std::to_string(v);
      for (uint64_t v : dims[i]) want += (want.empty() ? "" : ",") + std::to_string(v);
      return fail(CQ35_EINVAL, "GGUF tensor %s has shape [%s], expected [%s]", names[i].c_str(), got.c_str(),
                  want.c_str());
    }
    const uint32_t want_type = dtypes[i] == CQ35_BF16 ? gguf::kBF16 : gguf::kF32;
    if (t.type != want_type)
      return fail(CQ35_EINVAL, "GGUF tensor %s has dtype %u, expected %s", names[i].c_str(), t.type,
                  dtypes[i] == CQ35_BF16 ? "BF16" : "F32");
    uint64_t elements = 1;
    for (uint64_t v : t.dims) elements *= v;
    const uint64_t bytes = elements * (t.type == gguf::kF32 ? 4 : 2);
    const gguf::File& f = *ck.files[t.file];
    if (t.offset > f.size || bytes > f.size - t.offset)
      return fail(CQ35_EINVAL, "GGUF tensor %s range exceeds the length of %s", names[i].c_str(), f.path.c_str());
    ranges[t.file].emplace_back(t.offset, t.offset + bytes);
    (*pointers)[i] = f.base + t.offset;
  }
  for (size_t fi = 0; fi < ranges.size(); ++fi) {
    auto& r = ranges[fi];
    std::sort(r.begin(), r.end());
    r.erase(std::unique(r.begin(), r.end()), r.end());  // the tied head names the embedding again
    for (size_t k = 1; k < r.size(); ++k)
      if (r[k - 1].second > r[k].first)
        return fail(CQ35_EINVAL, "GGUF tensors overlap in %s", ck.files[fi]->path.c_str());
  }
  return CQ35_OK;
}

int gguf_open(const char* path, gguf::Checkpoint* ck) {
  if (!path) return fail(CQ35_EINVAL, "null path");
  std::string err;
  if (!gguf::open_all(path, ck, &err)) return fail(CQ35_EINVAL, "%s", err.c_str());
  return CQ35_OK;
}

}  // namespace

extern "C" int cq35_gguf_config(const char* path, cq35_config* out) {
  if (!out) return fail(CQ35_EINVAL, "null argument");
  gguf::Checkpoint ck;
  int rc = gguf_open(path, &ck);
  return rc ? rc : gguf_config_of(ck, out, nullptr);
}

extern "C" int cq35_gguf_validate(const char* path, const cq35_config* cfg) {
  gguf::Checkpoint ck;
  int rc = gguf_open(path, &ck);
  if (rc) return rc;
  cq35_config c;
  uint64_t nextn = 0;
  rc = gguf_config_of(ck, &c, &nextn);
  if (rc) return rc;
  if (cfg && std::memcmp(cfg, &c, sizeof c) != 0)
    return fail(CQ35_EINVAL, "the GGUF metadata describes a different configuration");
  std::vector<const void*> pointers;
  return gguf_check(ck, c, nextn, &pointers);
}

extern "C" int cq35_model_load_gguf(const char* path, cq35_model** out) {
  if (!out) return fail(CQ35_EINVAL, "null argument");
  gguf::Checkpoint ck;
  int rc = gguf_open(path, &ck);
  if (rc) return rc;
  cq35_config c;
  uint64_t nextn = 0;
  rc = gguf_config_of(ck, &c, &nextn);
  if (rc) return rc;
  std::vector<const void*> pointers;
  rc = gguf_check(ck, c, nextn, &pointers);
  if (rc) return rc;
  return cq35_model_create(&c, pointers.data(), 0, out);
}

extern "C" int cq35_gguf_tensor_name(const cq35_config* cfg, int64_t index, char* buf, int64_t len) {
  if (!cfg || !buf || len <= 0) return fail(CQ35_EINVAL, "null argument");
  std::string name;
  std::vector<uint64_t> dims;
  int32_t dt;
  if (!gguf_spec(*cfg, index, &name, &dims, &dt)) return fail(CQ35_ERANGE, "tensor index %lld out of range", (long long)index);
  if ((int64_t)name.size() + 1 > len) return fail(CQ35_EINVAL, "buffer too small for %s", name.c_str());
  std::memcpy(buf, name.c_str(), name.size() + 1);
  return CQ35_OK;
}

extern "C" int cq35_model_create_synthetic(const cq35_config* cfg, uint64_t seed, cq35_model** out) {
  int rc = cq35_config_validate(cfg);
  if (rc) return rc;
  if (!out) return fail(CQ35_EINVAL, "null argument");
  cq35_model* m = new (std::nothrow) cq35_model();
  if (!m) return fail(CQ35_EINVAL, "out of host memory");
  m->cfg = *cfg;
  m->d = dims_of(*cfg);
  hipGetDevice(&m->device);
  const int64_t n = weight_count(*cfg);
  m->w.assign(n, nullptr);
  for (int64_t i = 0; i < n; ++i) {
    TensorDesc t;
    describe(*cfg, i, &t);
    if (cfg->tied && i == n - 1) { m->w[i] = m->w[0]; continue; }  // lm_head = token_embd
    const int64_t bytes = tensor_bytes(t);
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
      cq35_model_free(m);
      return fail(CQ35_EDEVICE, "allocating weight %lld (%lld bytes): %s", (long long)i,
                  (long long)bytes, hipGetErrorString(e));
    }
    m->owned.push_back(p);
    m->w[i] = p;
    m->weight_bytes += bytes;
    const uint64_t key = mix64(seed ^ mix64((uint64_t)i + 1));
    float scale = normal_scale(0.02);
    if (t.kind == kConv) scale = normal_scale(0.3);
    if (t.kind == kRouter) scale = normal_scale(0.04);
    const int64_t count = t.rows * t.cols;
    const int blocks = (int)std::min<int64_t>((count + 255) / 256, 65536);
    k_fill<<<blocks, 256>>>(p, count, key, t.kind, scale);
    e = hipGetLastError();
    if (e != hipSuccess) {
      cq35_model_free(m);
      return fail(CQ35_EDEVICE, "synthetic fill of weight %lld: %s", (long long)i, hipGetErrorString(e));
    }
  }
  hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    cq35_model_free(m);
    return fail(CQ35_EDEVICE, "synthetic fill: %s", hipGetErrorString(e));
  }
  rc = finish_model(m);
  if (rc) { cq35_model_free(m); return rc; }
  *out = m;
  return CQ35_OK;
}

extern "C" int cq35_model_config(const cq35_model* m, cq35_config* out) {
  if (!m || !out) return fail(CQ35_EINVAL, "null argument");
  *out = m->cfg;
  return CQ35_OK;
}

extern "C" int cq35_model_weight_bytes(const cq35_model* m, int64_t* bytes) {
  if (!m || !bytes) return fail(CQ35_EINVAL, "null argument");
  *bytes = m->weight_bytes;
  return CQ35_OK;
}

extern "C" int cq35_model_read_weight(const cq35_model* m, int64_t index, void* dst, int64_t bytes) {
  if (!m || !dst) return fail(CQ35_EINVAL, "null argument");
  TensorDesc t;
  if (!describe(m->cfg, index, &t)) return fail(CQ35_EINVAL, "bad weight index");
  if (bytes != tensor_bytes(t)) return fail(CQ35_EINVAL, "size mismatch: tensor has %lld bytes", (long long)tensor_bytes(t));
  HIP_TRY(hipSetDevice(m->device));
  HIP_TRY(hipMemcpy(dst, m->w[index], bytes, hipMemcpyDeviceToHost));
  return CQ35_OK;
}

// ---------------------------------------------------------------- session

namespace {

// Launch classes for per-class event timing. RMSNorm is fused into the
// consuming GEMVs and top-k selection into the router, so neither has a class.
enum KernelClass {
  KC_EMBED = 0, KC_PROJECT, KC_PREPARE_LINEAR, KC_DELTA, KC_GATED_NORM, KC_RESIDUAL,
  KC_PREPARE_FULL, KC_ATTENTION, KC_ATTENTION_VALUES, KC_ROUTER, KC_MOE_GATE, KC_MOE_DOWN,
  KC_SWIGLU, KC_LOGITS, KC_SHADOW, KC_DECODE_STEP, KC_PREFILL_PROJECT, KC_COUNT
};
const char* kClassNames[KC_COUNT] = {
    "embed_rope", "project", "linear_prepare", "delta", "gated_norm", "residual_project",
    "full_prepare", "attention", "attention_values", "moe_router", "moe_gate_up", "moe_down",
    "swiglu", "logits_argmax", "shadow_copy", "decode_step", "prefill_project"};

constexpr int kMaxTimedEvents = 512;

}  // namespace

struct cq35_session {
  cq35_model* model = nullptr;
  int64_t capacity = 0;
  bool poisoned = false;
  hipStream_t stream = nullptr;
  // opaque state (reference layout)
  uint16_t* cache = nullptr;
  float* shadow = nullptr;
  // step parameters
  uint64_t* d_params = nullptr;
  uint64_t* h_params = nullptr;   // pinned
  unsigned long long* d_best = nullptr;
  unsigned long long* h_best = nullptr;  // pinned
  // activations
  uint16_t *h = nullptr, *attn = nullptr;
  uint16_t *qkv = nullptr, *conv = nullptr, *z = nullptr, *alpha = nullptr, *beta = nullptr;
  uint16_t *qn = nullptr, *kn = nullptr, *core = nullptr, *gated = nullptr;
  float2* gates = nullptr;  // per value head (decay, rate) of the current token
  uint16_t *qg = nullptr, *kraw = nullptr, *vraw = nullptr, *qr = nullptr, *ctx = nullptr;
  float* router = nullptr;
  int* ids = nullptr;
  float* probs = nullptr;
  unsigned* ticket = nullptr;  // router blocks finished (reset by the last one)
  uint16_t* active = nullptr;
  uint16_t* act = nullptr;
  uint16_t* logits = nullptr;
  float* rope = nullptr;
  float* attn_scratch = nullptr;
  int attn_stride = 0;
  std::vector<void*> allocations;
  // decode graph
  bool graph_enabled = true;
  hipGraph_t graph = nullptr;
  hipGraphExec_t graph_exec = nullptr;
  // persistent decode step (MoE): tagged exchange words, layer table, args
  bool mega_ok = false;       // the shape fits the persistent kernel
  bool mega_on = false;       // n == 1 steps use it
  bool mega_coop = false;     // launched cooperatively (co-residency of all blocks checked at launch)
  uint64_t* words = nullptr;
  MegaLayer* d_layers = nullptr;
  MegaArgs margs{};
  MegaArgs* d_margs = nullptr;
  int mega_grid = 0;
  const void* mega_kernel = nullptr;  // k_decode_step<shape> for this model
  int mega_lds = 0;                   // its dynamic LDS bytes
  uint32_t seq = 0;
  // batched prefill: chunk buffers of kBChunk token rows, allocated on the
  // first multi-token call at key_dim 128
  bool pf_ready = false;
  uint16_t *pf_h = nullptr, *pf_x = nullptr, *pf_attn = nullptr;
  uint16_t *pf_a = nullptr, *pf_b = nullptr, *pf_c = nullptr, *pf_d = nullptr;
  uint16_t *pf_e = nullptr, *pf_f = nullptr, *pf_g = nullptr, *pf_act = nullptr;
  float *pf_rope = nullptr, *pf_logits = nullptr, *pf_probs = nullptr, *pf_scratch = nullptr;
  float *pf_part = nullptr, *pf_spart = nullptr;  // matrix-core experts: routed / shared down sums
  int *pf_eoff = nullptr, *pf_order = nullptr;    // matrix-core experts: buckets
  int* pf_ids = nullptr;
  int pf_attn_tokens = 0;  // tokens per staged-attention launch (scratch rows)
  int pf_rows = 0;         // token rows of the chunk buffers
  int matrix = 0;          // CQ35_MATRIX_* components of multi-token calls on MFMA
  int matrix_decode = 0;   // weight-shared batched decode products on MFMA
  int64_t split_keys = CQ35_SPLIT_KEYS_DEFAULT;  // decode attention splits above this many keys
  // kernel timing
  int timed_class = -1;
  hipEvent_t ev[2 * kMaxTimedEvents] = {};
  int ev_used = 0;
  double timed_ms = 0.0;
  int64_t timed_launches = 0;
};

namespace {

template <typename T>
int dalloc(cq35_session* s, T** p, int64_t count) {
  void* q = nullptr;
  HIP_TRY(hipMalloc(&q, std::max<int64_t>(count, 1) * sizeof(T)));
  s->allocations.push_back(q);
  *p = static_cast<T*>(q);
  return CQ35_OK;
}

void destroy_session(cq35_session* s) {
  if (!s) return;
  hipSetDevice(s->model->device);
  if (s->stream) hipStreamSynchronize(s->stream);
  if (s->graph_exec) hipGraphExecDestroy(s->graph_exec);
  if (s->graph) hipGraphDestroy(s->graph);
  for (auto& e : s->ev) if (e) hipEventDestroy(e);
  for (void* p : s->allocations) hipFree(p);
  if (s->h_params) hipHostFree(s->h_params);
  if (s->h_best) hipHostFree(s->h_best);
  if (s->stream) hipStreamDestroy(s->stream);
  delete s;
}

// Model shapes the persistent decode kernels are compiled for (mega.h for
// the MoE shapes, dense_step.h for the dense ones) and the per-grid limits of
// their work split; other shapes and capacities use the per-kernel path.
// Returns the shape index (0 = none).
enum MegaKind {
  kMegaNone = 0, kMega35B, kMegaMini, kMegaTiny,
  kDense2B, kDense08B, kDenseMini, kDenseTiny
};

template <class S>
bool shape_is(const cq35_config& c) {
  return c.moe && c.hidden == S::H && c.vocab == S::V && c.q_heads == S::Q && c.kv_heads == S::KVH &&
         c.head_dim == S::HD && c.rope_dim == S::R && c.key_heads == S::KH && c.key_dim == S::KD &&
         c.value_heads == S::VH && c.value_dim == S::VD && c.experts == S::E && c.top_k == S::K &&
         c.intermediate == S::I && c.shared_intermediate == S::SI;
}

template <class S>
bool grid_fits(int grid) {
  const int64_t nw = (int64_t)grid * kMW;
  const int64_t rows_lin = S::QKV + S::VS, rows_full = 2LL * S::QS + 2LL * S::KVS;
  return S::VH <= grid && std::max(rows_lin, rows_full) / 2 <= kPairsA * nw && S::H / 2 <= (int64_t)(kMW / 2) * grid &&
         S::H / 2 <= (int64_t)DownLayout<S>::WAVES * grid &&
         S::K * S::I / 2 <= nw && S::E + 1 <= (int64_t)(kMW / 2) * grid &&
         S::SI / 2 <= grid && S::H / 2 <= nw;
}

template <class S>
bool dense_shape_is(const cq35_config& c) {
  return !c.moe && c.hidden == S::H && c.vocab == S::V && c.q_heads == S::Q && c.kv_heads == S::KVH &&
         c.head_dim == S::HD && c.rope_dim == S::R && c.key_heads == S::KH && c.key_dim == S::KD &&
         c.value_heads == S::VH && c.value_dim == S::VD && c.intermediate == S::I;
}

template <class S>
bool dense_grid_fits(int grid) {
  return S::VH <= grid && S::Q <= grid && S::H / 2 <= (int64_t)(kMW / 2) * grid &&
         S::I <= (int64_t)kDenseFfnRows * kMW * grid;
}

int mega_kind(const cq35_config& c, int grid) {
  if (dense_shape_is<ShapeDense2B>(c)) return dense_grid_fits<ShapeDense2B>(grid) ? kDense2B : kMegaNone;
  if (dense_shape_is<ShapeDense08B>(c)) return dense_grid_fits<ShapeDense08B>(grid) ? kDense08B : kMegaNone;
  if (dense_shape_is<ShapeDenseMini>(c)) return dense_grid_fits<ShapeDenseMini>(grid) ? kDenseMini : kMegaNone;
  if (dense_shape_is<ShapeDenseTiny>(c)) return dense_grid_fits<ShapeDenseTiny>(grid) ? kDenseTiny : kMegaNone;
  if (shape_is<Shape35BA3B>(c)) return grid_fits<Shape35BA3B>(grid) ? kMega35B : kMegaNone;
  if (shape_is<ShapeMiniMoE>(c)) return grid_fits<ShapeMiniMoE>(grid) ? kMegaMini : kMegaNone;
  if (shape_is<ShapeTinyMoE>(c)) return grid_fits<ShapeTinyMoE>(grid) ? kMegaTiny : kMegaNone;
  return kMegaNone;
}

int mega_lds(int kind) {
  switch (kind) {
    case kMega35B: return mega_lds_request<Shape35BA3B>();
    case kMegaMini: return mega_lds_request<ShapeMiniMoE>();
    case kMegaTiny: return mega_lds_request<ShapeTinyMoE>();
    case kDense2B: return dense_lds_request<ShapeDense2B>();
    case kDense08B: return dense_lds_request<ShapeDense08B>();
    case kDenseMini: return dense_lds_request<ShapeDenseMini>();
    case kDenseTiny: return dense_lds_request<ShapeDenseTiny>();
    default: return 0;
  }
}

const void* mega_kernel(int kind) {
  switch (kind) {
    case kMega35B: return (const void*)k_decode_step<Shape35BA3B>;
    case kMegaMini: return (const void*)k_decode_step<ShapeMiniMoE>;
    case kMegaTiny: return (const void*)k_decode_step<ShapeTinyMoE>;
    case kDense2B: return (const void*)k_dense_step<ShapeDense2B>;
    case kDense08B: return (const void*)k_dense_step<ShapeDense08B>;
    case kDenseMini: return (const void*)k_dense_step<ShapeDenseMini>;
    case kDenseTiny: return (const void*)k_dense_step<ShapeDenseTiny>;
    default: return nullptr;
  }
}

// Tagged exchange buffers per layer (each region 128-byte aligned), the
// device layer table and the kernel arguments of the persistent step.
int setup_mega(cq35_session* s) {
  const cq35_model& m = *s->model;
  const cq35_config& c = m.cfg;
  const Dims& d = m.d;
  int grid = 0;
  HIP_TRY(hipDeviceGetAttribute(&grid, hipDeviceAttributeMultiprocessorCount, m.device));
  const int kind = mega_kind(c, grid);
  const void* kernel = mega_kernel(kind);
  if (!kernel) return CQ35_OK;
  const bool dense = !c.moe;
  if (dense && s->capacity > kDenseKeys) return CQ35_OK;  // the softmax phase holds a head's scores in LDS
  const int lds = mega_lds(kind);
  if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, lds) != hipSuccess)
    return CQ35_OK;
  int occupancy = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occupancy, kernel, kMT, lds) != hipSuccess ||
      occupancy < 1)
    return CQ35_OK;
  auto region = [](int64_t words) { return (words + 15) / 16 * 16; };
  const int64_t hw = region(d.H / 2);
  // per layer: h, proj, mix, attn, router, active, scores, shared
  std::vector<int64_t> offs;
  int64_t total = 0;
  for (int64_t l = 0; l < d.L; ++l) {
    const bool full = is_full(c, l);
    // dense linear layers also project alpha and beta (S32 rows)
    const int64_t proj = full ? 2 * d.QS + 2 * d.KVS : d.QKV + d.VS + (dense ? 2 * c.value_heads : 0);
    // full layers: Q x capacity score words, or (split-K) per query head and
    // range the partial words (m, den, acc[HD])
    const int64_t scores = std::max<int64_t>(d.Q * s->capacity, d.Q * kSplitRanges * (2 + d.HD));
    const int64_t sizes[8] = {hw, region(proj / 2), region((full ? d.QS : d.VS) / 2), hw,
                              dense ? 0 : region(d.E + 1),
                              region(dense ? d.I / 2 : d.K * d.I / 2),
                              full ? region(scores) : 0, dense ? 0 : region(d.SI / 2)};
    for (int64_t z : sizes) {
      offs.push_back(total);
      total += z;
    }
  }
  const int64_t final_off = total;
  total += hw;
  void* p = nullptr;
  HIP_TRY(hipMalloc(&p, total * sizeof(uint64_t)));
  s->allocations.push_back(p);
  s->words = static_cast<uint64_t*>(p);
  HIP_TRY(hipMemset(s->words, 0, total * sizeof(uint64_t)));
  std::vector<MegaLayer> layers(d.L);
  int64_t base = 1;
  const int64_t cap = s->capacity;
  for (int64_t l = 0; l < d.L; ++l) {
    auto W = [&](int slot) { return m.w[base + slot]; };
    MegaLayer& Ly = layers[l];
    Ly = MegaLayer{};
    const int64_t* o = &offs[8 * l];
    Ly.full = is_full(c, l) ? 1 : 0;
    Ly.in_norm = (const float*)W(0);
    Ly.x_h = s->words + o[0];
    Ly.x_proj = s->words + o[1];
    Ly.x_mix = s->words + o[2];
    Ly.x_attn = s->words + o[3];
    Ly.x_router = dense ? nullptr : s->words + o[4];
    Ly.x_active = s->words + o[5];
    Ly.x_scores = s->words + o[6];
    Ly.x_shared = s->words + o[7];
    Ly.x_out = l + 1 < d.L ? s->words + offs[8 * (l + 1)] : s->words + final_off;
    int ffn;
    if (Ly.full) {
      Ly.seg_w[0] = (const uint16_t*)W(1); Ly.seg_rows[0] = (int)(2 * d.QS);
      Ly.seg_w[1] = (const uint16_t*)W(2); Ly.seg_rows[1] = (int)d.KVS;
      Ly.seg_w[2] = (const uint16_t*)W(3); Ly.seg_rows[2] = (int)d.KVS;
      Ly.out_w = (const uint16_t*)W(4);
      Ly.qnorm = (const float*)W(5);
      Ly.knorm = (const float*)W(6);
      Ly.post_norm = (const float*)W(7);
      Ly.key_base = l * 2 * cap * d.KVS;
      Ly.value_base = Ly.key_base + cap * d.KVS;
      ffn = 8;
    } else {
      Ly.seg_w[0] = (const uint16_t*)W(1); Ly.seg_rows[0] = (int)d.QKV;
      Ly.seg_w[1] = (const uint16_t*)W(2); Ly.seg_rows[1] = (int)d.VS;
      if (dense) {
        Ly.seg_w[2] = (const uint16_t*)W(3); Ly.seg_rows[2] = c.value_heads;
        Ly.seg_w[3] = (const uint16_t*)W(4); Ly.seg_rows[3] = c.value_heads;
      }
      Ly.alpha_w = (const uint16_t*)W(3);
      Ly.beta_w = (const uint16_t*)W(4);
      Ly.dt = (const float*)W(5);
      Ly.a = (const float*)W(6);
      Ly.gnorm = (const float*)W(7);
      Ly.out_w = (const uint16_t*)W(8);
      Ly.conv_w = (const float*)W(9);
      Ly.post_norm = (const float*)W(10);
      Ly.conv_base = cap * d.KV_STRIDE + l * d.LIN;
      Ly.state_base = Ly.conv_base + d.CONV;
      ffn = 11;
    }
    if (dense) {
      // the dense SwiGLU in the shared-expert slots: gate, up, down
      Ly.sgate = (const uint16_t*)W(ffn);
      Ly.sup = (const uint16_t*)W(ffn + 1);
      Ly.sdown = (const uint16_t*)W(ffn + 2);
    } else {
      Ly.router = (const float*)W(ffn);
      Ly.gate_exps = (const uint16_t*)W(ffn + 1);
      Ly.up_exps = (const uint16_t*)W(ffn + 2);
      Ly.down_exps = (const uint16_t*)W(ffn + 3);
      Ly.shared_gate = (const float*)W(ffn + 4);
      Ly.sgate = (const uint16_t*)W(ffn + 5);
      Ly.sup = (const uint16_t*)W(ffn + 6);
      Ly.sdown = (const uint16_t*)W(ffn + 7);
    }
    base += layer_tensors(c, l);
  }
  p = nullptr;
  HIP_TRY(hipMalloc(&p, layers.size() * sizeof(MegaLayer)));
  s->allocations.push_back(p);
  s->d_layers = static_cast<MegaLayer*>(p);
  HIP_TRY(hipMemcpy(s->d_layers, layers.data(), layers.size() * sizeof(MegaLayer), hipMemcpyHostToDevice));
  MegaArgs& a = s->margs;
  a = MegaArgs{};
  a.layers = s->d_layers;
  a.L = (int)d.L;
  a.eps = c.eps;
  a.attn_scale = 1.0f / sqrtf((float)d.HD);        // SCALE_BITS, qwen35.rs:701
  a.delta_scale = 1.0f / sqrtf((float)c.key_dim);  // DELTA_SCALE_BITS, qwen35.rs:703
  a.cap = cap;
  const int64_t nweights = weight_count(c);
  a.embed = (const uint16_t*)m.w[0];
  a.out_norm = (const float*)m.w[nweights - 2];
  a.head = (const uint16_t*)m.w[nweights - 1];
  a.freq = m.freq;
  a.cache = s->cache;
  a.params = s->d_params;
  a.x_final = s->words + final_off;
  a.logits = s->logits;
  a.best = s->d_best;
  a.error = reinterpret_cast<unsigned*>(s->d_best + 1);
  a.ids_out = s->ids;
  a.split_keys = s->split_keys;
  a.spin_limit = 1u << 21;
#ifdef CQ35_PHASE_TRACE
  p = nullptr;
  HIP_TRY(hipMalloc(&p, (size_t)grid * kTraceSlots * sizeof(uint64_t)));
  s->allocations.push_back(p);
  a.trace = static_cast<uint64_t*>(p);
#endif
  if (const char* lim = getenv("CQ35_SPIN_LIMIT")) a.spin_limit = (unsigned)strtoul(lim, nullptr, 10);
  p = nullptr;
  HIP_TRY(hipMalloc(&p, sizeof(MegaArgs)));
  s->allocations.push_back(p);
  s->d_margs = static_cast<MegaArgs*>(p);
  HIP_TRY(hipMemcpy(s->d_margs, &a, sizeof(MegaArgs), hipMemcpyHostToDevice));
  s->mega_grid = grid;
  s->mega_kernel = kernel;
  s->mega_lds = lds;
  // Every block waits on others' words, so all of them must be resident at
  // once: a cooperative launch has the runtime check that (and fail the
  // launch) instead of leaving it to the occupancy computed above.
  // CQ35_COOPERATIVE=0 selects the ordinary launch.
  int coop = 0;
  hipDeviceGetAttribute(&coop, hipDeviceAttributeCooperativeLaunch, m.device);
  s->mega_coop = coop != 0;
  if (const char* cl = getenv("CQ35_COOPERATIVE")) s->mega_coop = s->mega_coop && atoi(cl) != 0;
  s->mega_ok = true;
  s->mega_on = true;
  if (const char* g = getenv("CQ35_PERSISTENT")) s->mega_on = atoi(g) != 0;
  return CQ35_OK;
}

int create_session(cq35_model* m, int64_t capacity, cq35_session** out) {
  cq35_session* s = new (std::nothrow) cq35_session();
  if (!s) return fail(CQ35_EINVAL, "out of host memory");
  s->model = m;
  s->capacity = capacity;
  const Dims& d = m->d;
  const cq35_config& c = m->cfg;
  int rc = CQ35_OK;
  auto check = [&](int r) { if (r && !rc) rc = r; };
  hipError_t e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
  if (e != hipSuccess) { destroy_session(s); return fail(CQ35_EDEVICE, "stream: %s", hipGetErrorString(e)); }
  const int64_t cache_n = cache_elements(c, capacity);
  check(dalloc(s, &s->cache, cache_n));
  check(dalloc(s, &s->shadow, d.L * d.REC));
  check(dalloc(s, &s->d_params, capacity + 2));
  check(dalloc(s, &s->d_best, 2));  // [0] argmax key, [1] persistent-kernel error word
  check(dalloc(s, &s->h, d.H));
  check(dalloc(s, &s->attn, d.H));
  check(dalloc(s, &s->qkv, d.QKV));
  check(dalloc(s, &s->conv, d.QKV));
  check(dalloc(s, &s->z, d.VS));
  check(dalloc(s, &s->alpha, c.value_heads));
  check(dalloc(s, &s->beta, c.value_heads));
  check(dalloc(s, &s->qn, d.KS));
  check(dalloc(s, &s->gates, c.value_heads));
  check(dalloc(s, &s->kn, d.KS));
  check(dalloc(s, &s->core, d.VS));
  check(dalloc(s, &s->gated, d.VS));
  check(dalloc(s, &s->qg, 2 * d.QS));
  check(dalloc(s, &s->kraw, d.KVS));
  check(dalloc(s, &s->vraw, d.KVS));
  check(dalloc(s, &s->qr, d.QS));
  check(dalloc(s, &s->ctx, d.QS));
  check(dalloc(s, &s->router, d.E + 1));
  check(dalloc(s, &s->ids, d.L * std::max<int64_t>(d.K, 1)));  // per layer: the last token's top-k
  check(dalloc(s, &s->probs, std::max<int64_t>(d.K, 1)));
  check(dalloc(s, &s->ticket, 1));
  check(dalloc(s, &s->active, d.K * d.I + d.SI));
  check(dalloc(s, &s->act, d.I));
  check(dalloc(s, &s->logits, d.V));
  check(dalloc(s, &s->rope, std::max<int64_t>(d.R, 2)));
  // online: scores/weights (tiles*8) + running max + alpha (tiles each);
  // staged: scores + exponentials (keys each) + BF16 weights.
  const int64_t tiles = (capacity + 7) / 8;
  s->attn_stride = (int)std::max<int64_t>(tiles * 8 + 2 * tiles + 16, 3 * capacity + 16);
  check(dalloc(s, &s->attn_scratch, d.Q * (int64_t)s->attn_stride));
  if (rc) { destroy_session(s); return rc; }
  if (const char* g = getenv("CQ35_GRAPH")) s->graph_enabled = atoi(g) != 0;
  e = hipHostMalloc((void**)&s->h_params, (capacity + 2) * sizeof(uint64_t), hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void**)&s->h_best, 2 * sizeof(unsigned long long), hipHostMallocDefault);
  if (e == hipSuccess) e = hipMemset(s->cache, 0, cache_n * sizeof(uint16_t));
  if (e == hipSuccess) e = hipMemset(s->shadow, 0, d.L * d.REC * sizeof(float));
  if (e == hipSuccess) e = hipMemset(s->ticket, 0, sizeof(unsigned));
  if (e == hipSuccess) e = hipMemset(s->d_best, 0, 2 * sizeof(unsigned long long));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) { destroy_session(s); return fail(CQ35_EDEVICE, "session init: %s", hipGetErrorString(e)); }
  rc = setup_mega(s);
  if (rc) { destroy_session(s); return rc; }
  *out = s;
  return CQ35_OK;
}

// ---------------------------------------------------------- launch helpers

struct Launcher {
  cq35_session* s;
  template <typename Kernel, typename... Args>
  void operator()(int kc, Kernel kernel, dim3 grid, dim3 block, size_t lds, Args... args) {
    const bool timed = s->timed_class == kc && s->ev_used < kMaxTimedEvents;
    if (timed) {
      // Events stamped by the dispatch packet itself, so the interval is the
      // kernel's execution as a profiler sees it, without event-record gaps.
      hipExtLaunchKernelGGL(kernel, grid, block, (uint32_t)lds, s->stream, s->ev[2 * s->ev_used],
                            s->ev[2 * s->ev_used + 1], 0, args...);
      ++s->ev_used;
    } else {
      kernel<<<grid, block, lds, s->stream>>>(args...);
    }
  }
};

int grid_for(int64_t groups, int64_t cap) { return (int)std::max<int64_t>(1, std::min(groups, cap)); }

int64_t seg_rows(const Segments& seg) {
  return (int64_t)seg.rows[0] + seg.rows[1] + seg.rows[2] + seg.rows[3];
}

// Register batch (quads, or dwords for the router) per lane: the smallest
// instantiated size that covers `per_lane`, capped at the largest.
int batch_of(int64_t per_lane, std::initializer_list<int> sizes) {
  int pick = 0;
  for (int n : sizes) {
    pick = n;
    if (per_lane <= n) break;
  }
  return pick;
}

// S256 grouped projection of the normalised hidden row (MoE models).
void project256(Launcher& L, int kc, const uint16_t* x, const float* norm_w, float eps,
                const Segments& seg, int64_t cols) {
  const int64_t per_block = 4 * kRows256;
  L(kc, k_project256<true>, dim3((unsigned)((seg_rows(seg) + per_block - 1) / per_block)),
    dim3(kBlock), (size_t)cols * 2, x, norm_w, eps, seg, (int)cols);
}

// S32 projection of the normalised hidden row (dense models) and, with
// kArgmax, the vocabulary head with the fused greedy argmax.
template <bool kArgmax>
void project32(Launcher& L, int kc, const uint16_t* x, const float* norm_w, float eps,
               const Segments& seg, int64_t cols, unsigned long long* best) {
  const dim3 grid((unsigned)((seg_rows(seg) + 31) / 32)), block(kBlock);
  const size_t lds = (size_t)cols * 2;
  switch (batch_of((cols / 8 + 7) / 8, {8, 16, 32})) {
    case 8: L(kc, k_project32<true, kArgmax, 8>, grid, block, lds, x, norm_w, eps, seg, (int)cols, best); break;
    case 16: L(kc, k_project32<true, kArgmax, 16>, grid, block, lds, x, norm_w, eps, seg, (int)cols, best); break;
    default: L(kc, k_project32<true, kArgmax, 32>, grid, block, lds, x, norm_w, eps, seg, (int)cols, best); break;
  }
}

// bf16(bf16(tree64(x . w_r)) (+) res_r) for the hidden-width outputs
// (qwen3.fused.residual, simt.hex:442-538).
void residual(Launcher& L, const uint16_t* x, const void* w, int64_t rows, int64_t cols,
              const uint16_t* res, uint16_t* out) {
  const dim3 grid((unsigned)((rows + 3) / 4)), block(64);
  const size_t lds = (size_t)cols * 2;
  const uint16_t* wq = static_cast<const uint16_t*>(w);
  switch (batch_of((cols / 8 + 15) / 16, {8, 16, 32})) {
    case 8: L(KC_RESIDUAL, k_residual<8>, grid, block, lds, x, wq, (int)rows, (int)cols, res, out); break;
    case 16: L(KC_RESIDUAL, k_residual<16>, grid, block, lds, x, wq, (int)rows, (int)cols, res, out); break;
    default: L(KC_RESIDUAL, k_residual<32>, grid, block, lds, x, wq, (int)rows, (int)cols, res, out); break;
  }
}

// MoE router + top-k selection (one launch; the last block selects).
void router_select(Launcher& L, cq35_session* s, int64_t layer, const uint16_t* x, const float* norm_w,
                   const float* w, const float* shared_w) {
  const Dims& d = s->model->d;
  int* ids = s->ids + layer * d.K;
  const float eps = s->model->cfg.eps;
  const dim3 grid((unsigned)((d.E + 1 + 3) / 4)), block(kBlock);
  const size_t lds = router_lds_bytes((int)d.H, (int)d.E);
  switch (batch_of((d.H + 63) / 64, {8, 16, 32})) {
    case 8: L(KC_ROUTER, k_router_select<8>, grid, block, lds, x, norm_w, eps, (int)d.H, w, shared_w, (int)d.E, (int)d.K, s->router, ids, s->probs, s->ticket); break;
    case 16: L(KC_ROUTER, k_router_select<16>, grid, block, lds, x, norm_w, eps, (int)d.H, w, shared_w, (int)d.E, (int)d.K, s->router, ids, s->probs, s->ticket); break;
    default: L(KC_ROUTER, k_router_select<32>, grid, block, lds, x, norm_w, eps, (int)d.H, w, shared_w, (int)d.E, (int)d.K, s->router, ids, s->probs, s->ticket); break;
  }
}

int down_batch(const Dims& d) { return batch_of(((d.K * d.I + d.SI) / 8 + 63) / 64, {4, 8, 12, 16, 24}); }

// Expert down projection + residual + shared expert.
void moe_down(Launcher& L, cq35_session* s, int64_t layer, const void* down, const void* sdown) {
  const Dims& d = s->model->d;
  const int* ids = s->ids + layer * d.K;
  const int per_row = (int)((d.K * d.I + d.SI) / 8);
  const dim3 grid((unsigned)((d.H + kDownRows - 1) / kDownRows)), block(kBlock);
  const size_t lds = moe_down_lds_bytes(per_row);
  const uint16_t* dw = static_cast<const uint16_t*>(down);
  const uint16_t* sw = static_cast<const uint16_t*>(sdown);
  const int H = (int)d.H, K = (int)d.K, I = (int)d.I, SI = (int)d.SI;
  switch (down_batch(d)) {
    case 4: L(KC_MOE_DOWN, k_moe_down<4>, grid, block, lds, (const uint16_t*)s->active, dw, sw, ids, (const uint16_t*)s->attn, H, K, I, SI, s->h); break;
    case 8: L(KC_MOE_DOWN, k_moe_down<8>, grid, block, lds, (const uint16_t*)s->active, dw, sw, ids, (const uint16_t*)s->attn, H, K, I, SI, s->h); break;
    case 12: L(KC_MOE_DOWN, k_moe_down<12>, grid, block, lds, (const uint16_t*)s->active, dw, sw, ids, (const uint16_t*)s->attn, H, K, I, SI, s->h); break;
    case 16: L(KC_MOE_DOWN, k_moe_down<16>, grid, block, lds, (const uint16_t*)s->active, dw, sw, ids, (const uint16_t*)s->attn, H, K, I, SI, s->h); break;
    default: L(KC_MOE_DOWN, k_moe_down<24>, grid, block, lds, (const uint16_t*)s->active, dw, sw, ids, (const uint16_t*)s->attn, H, K, I, SI, s->h); break;
  }
}

// Largest dynamic LDS of the MoE down kernel; above 64 KiB the kernel must
// be opted in.
hipError_t moe_down_lds_optin(const Dims& d) {
  const size_t lds = moe_down_lds_bytes((int)((d.K * d.I + d.SI) / 8));
  if (lds <= 65536) return hipSuccess;
  const void* f = nullptr;
  switch (down_batch(d)) {
    case 4: f = (const void*)k_moe_down<4>; break;
    case 8: f = (const void*)k_moe_down<8>; break;
    case 12: f = (const void*)k_moe_down<12>; break;
    case 16: f = (const void*)k_moe_down<16>; break;
    default: f = (const void*)k_moe_down<24>; break;
  }
  return hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
}

Segments segments(std::initializer_list<std::pair<const void*, std::pair<uint16_t*, int64_t>>> list) {
  Segments s{};
  int i = 0;
  for (auto& e : list) {
    s.w[i] = static_cast<const uint16_t*>(e.first);
    s.out[i] = e.second.first;
    s.rows[i] = (int)e.second.second;
    ++i;
  }
  s.count = i;
  return s;
}

// Enqueue token t of the call: embedding, every layer, and (for the last
// token) the head. f32_state selects the F32 shadow DeltaNet state used
// inside a multi-token call (cached_delta.hex:230-261).
void enqueue_token(cq35_session* s, int t, bool last, bool f32_state) {
  const cq35_model& m = *s->model;
  const cq35_config& c = m.cfg;
  const Dims& d = m.d;
  Launcher L{s};
  auto Wt = [&](int64_t index) { return m.w[index]; };
  const int64_t cap = s->capacity;
  L(KC_EMBED, k_embed, dim3(grid_for((d.H + kBlock - 1) / kBlock, 64)), dim3(kBlock), 0,
    (const uint64_t*)s->d_params, t, (const uint16_t*)Wt(0), (int)d.H, s->h, (const float*)m.freq,
    (int)(d.R / 2), s->rope, last ? s->d_best : (unsigned long long*)nullptr);
  int64_t base = 1;
  for (int64_t l = 0; l < d.L; ++l) {
    auto W = [&](int slot) { return Wt(base + slot); };
    const int64_t key_base = l * 2 * cap * d.KVS;
    const int64_t value_base = key_base + cap * d.KVS;
    const float* in_norm = (const float*)W(0);
    auto project = [&](const Segments& seg) {
      if (c.moe) project256(L, KC_PROJECT, s->h, in_norm, c.eps, seg, d.H);
      else project32<false>(L, KC_PROJECT, s->h, in_norm, c.eps, seg, d.H, nullptr);
    };
    int ffn;
    const float* post_norm;
    if (is_full(c, l)) {
      project(segments({{W(1), {s->qg, 2 * d.QS}}, {W(2), {s->kraw, d.KVS}}, {W(3), {s->vraw, d.KVS}}}));
      L(KC_PREPARE_FULL, k_full_prepare, dim3((unsigned)(d.Q + d.KVH)), dim3(kBlock), 0,
        (const uint16_t*)s->qg, (const uint16_t*)s->kraw, (const uint16_t*)s->vraw,
        (const float*)s->rope, (const float*)W(5), (const float*)W(6), s->cache, key_base,
        value_base, (const uint64_t*)s->d_params, t, (int)d.KVS, (int)d.Q, (int)d.HD, d.pad_hd,
        (int)d.R, c.eps, s->qr, (const SessionRows*)nullptr);
      const float scale = 1.0f / sqrtf((float)d.HD);  // SCALE_BITS, qwen35.rs:701
      if (c.moe) {
        L(KC_ATTENTION, k_attn_scores,
          dim3((unsigned)std::min<int64_t>((cap + 7) / 8, 512), (unsigned)d.KVH), dim3(kScoreBlock),
          (size_t)(d.Q / d.KVH) * d.HD * 4, (const uint16_t*)s->qr, (const uint16_t*)s->cache,
          key_base, (const uint64_t*)s->d_params, t, (int)d.KVS, (int)d.HD, (int)(d.Q / d.KVH),
          scale, s->attn_scratch, s->attn_stride, (const SessionRows*)nullptr);
        L(KC_ATTENTION_VALUES, k_attn_values,
          dim3((unsigned)d.Q, (unsigned)((d.HD + kValueChannels - 1) / kValueChannels)), dim3(64),
          attn_values_lds_bytes(cap), (const float*)s->attn_scratch,
          s->attn_stride, (const uint16_t*)s->cache, value_base, (const uint64_t*)s->d_params, t,
          (int)d.KVS, (int)d.HD, (int)(d.Q / d.KVH), (const uint16_t*)s->qg, s->split_keys, s->ctx);
      } else {
        // regrouped (scores per key chunk and head pair, the softmax, the
        // context per KV head) where the shape allows; the scores grid covers
        // the capacity, since a captured graph replays at later positions
        const int hpk = (int)(d.Q / d.KVH);
        const bool regroup = d.HD % 8 == 0 && d.HD <= 256 && (hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8);
        const uint64_t* params = (const uint64_t*)s->d_params;
        if (regroup) {
          const unsigned chunks = (unsigned)((cap + 255) / 256);
          if (hpk % 2 == 0)
            L(KC_ATTENTION, k_bstaged_scores<2>, dim3(chunks, (unsigned)(d.KVH * hpk / 2)), dim3(256), 0,
              (const uint16_t*)s->qr, (const SessionRows*)nullptr, (const uint16_t*)s->cache, params, t, key_base,
              (int)d.KVS, (int)d.HD, (int)d.Q, hpk, scale, s->attn_scratch, s->attn_stride);
          else
            L(KC_ATTENTION, k_bstaged_scores<1>, dim3(chunks, (unsigned)(d.KVH * hpk)), dim3(256), 0,
              (const uint16_t*)s->qr, (const SessionRows*)nullptr, (const uint16_t*)s->cache, params, t, key_base,
              (int)d.KVS, (int)d.HD, (int)d.Q, hpk, scale, s->attn_scratch, s->attn_stride);
        }
        L(KC_ATTENTION, k_attention_staged, dim3((unsigned)d.Q), dim3(kStagedThreads), 0,
          (const uint16_t*)s->qr, (const uint16_t*)s->cache, key_base, params, t,
          (int)d.KVS, (int)d.HD, hpk, scale, s->attn_scratch, s->attn_stride, (const SessionRows*)nullptr,
          regroup);
        const dim3 cgrid((unsigned)(d.KVH * d.HD / kContextChannels));
        auto grouped = [&](auto kernel) {
          L(KC_ATTENTION, kernel, cgrid, dim3(kContextThreads), 0, (const uint16_t*)s->cache, params, t, value_base,
            (int)d.KVS, (int)d.HD, (int)d.Q, (const uint16_t*)s->qg, (const float*)s->attn_scratch, s->attn_stride,
            s->ctx, (const SessionRows*)nullptr);
        };
        if (regroup && hpk == 1) grouped(k_battention_context<1>);
        else if (regroup && hpk == 2) grouped(k_battention_context<2>);
        else if (regroup && hpk == 4) grouped(k_battention_context<4>);
        else if (regroup && hpk == 8) grouped(k_battention_context<8>);
        else
          L(KC_ATTENTION, k_attention_context, dim3((unsigned)(d.Q * d.HD / kContextChannels)), dim3(kContextThreads),
            0, (const uint16_t*)s->cache, value_base, params, t, (int)d.KVS, (int)d.HD, (int)d.Q, hpk,
            (const uint16_t*)s->qg, (const float*)s->attn_scratch, s->attn_stride, s->ctx, (const SessionRows*)nullptr);
      }
      residual(L, s->ctx, W(4), d.H, d.QS, s->h, s->attn);
      post_norm = (const float*)W(7);
      ffn = 8;
    } else {
      project(segments({{W(1), {s->qkv, d.QKV}}, {W(2), {s->z, d.VS}},
                        {W(3), {s->alpha, c.value_heads}}, {W(4), {s->beta, c.value_heads}}}));
      const int64_t conv_base = cap * d.KV_STRIDE + l * d.LIN;
      L(KC_PREPARE_LINEAR, k_linear_prepare, dim3((unsigned)((d.QKV + c.key_dim - 1) / c.key_dim)),
        dim3(kBlock), 0, (const uint16_t*)s->qkv, s->cache, conv_base, (const uint64_t*)s->d_params,
        t, (const float*)W(9), (int)d.QKV, c.key_dim, c.key_heads, s->conv, s->qn, s->kn, (const SessionRows*)nullptr,
        (const uint16_t*)s->alpha, (const uint16_t*)s->beta, (const float*)W(5), (const float*)W(6), c.value_heads,
        s->gates);
      const float scale = 1.0f / sqrtf((float)c.key_dim);  // DELTA_SCALE_BITS, qwen35.rs:703
      const dim3 dgrid((unsigned)((d.VS + 8 * kDeltaCh - 1) / (8 * kDeltaCh)));
      const bool kd128 = c.key_dim == 128;
      if (f32_state)
        L(KC_DELTA, kd128 ? k_delta<true, 128> : k_delta<true, 0>, dgrid, dim3(kBlock), 0, (const uint16_t*)s->conv,
          (const uint16_t*)s->qn, (const uint16_t*)s->kn, (const float2*)s->gates, (uint16_t*)nullptr,
          s->shadow + l * d.REC, (int)d.VS, c.value_dim, c.key_dim, c.key_heads, (int)d.KS, scale,
          s->core, (const SessionRows*)nullptr, (int64_t)0);
      else
        L(KC_DELTA, kd128 ? k_delta<false, 128> : k_delta<false, 0>, dgrid, dim3(kBlock), 0, (const uint16_t*)s->conv,
          (const uint16_t*)s->qn, (const uint16_t*)s->kn, (const float2*)s->gates,
          s->cache + conv_base + d.CONV, (float*)nullptr, (int)d.VS, c.value_dim, c.key_dim,
          c.key_heads, (int)d.KS, scale, s->core, (const SessionRows*)nullptr, (int64_t)0);
      L(KC_GATED_NORM, k_gated_norm, dim3((unsigned)c.value_heads), dim3(kBlock), 0,
        (const uint16_t*)s->core, (const uint16_t*)s->z, (const float*)W(7), c.value_dim, c.eps,
        s->gated);
      residual(L, s->gated, W(8), d.H, d.VS, s->h, s->attn);
      post_norm = (const float*)W(10);
      ffn = 11;
    }
    if (c.moe) {
      router_select(L, s, l, s->attn, post_norm, (const float*)W(ffn), (const float*)W(ffn + 4));
      const int64_t rows = d.K * d.I + d.SI;
      L(KC_MOE_GATE, k_gate_up<true>, dim3((unsigned)((rows + 4 * kRowsGate - 1) / (4 * kRowsGate))),
        dim3(kBlock), (size_t)d.H * 2, (const uint16_t*)s->attn, post_norm, c.eps, (int)d.H,
        (const uint16_t*)W(ffn + 1), (const uint16_t*)W(ffn + 2), (const uint16_t*)W(ffn + 5),
        (const uint16_t*)W(ffn + 6), (const int*)(s->ids + l * d.K), (const float*)s->probs,
        (const float*)s->router, (int)d.E, (int)d.K, (int)d.I, (int)d.SI, s->active);
      moe_down(L, s, l, W(ffn + 3), W(ffn + 7));
    } else {
      L(KC_SWIGLU, k_gate_up<false>, dim3((unsigned)((d.I + 4 * kRowsGate - 1) / (4 * kRowsGate))),
        dim3(kBlock), (size_t)d.H * 2, (const uint16_t*)s->attn, post_norm, c.eps, (int)d.H,
        (const uint16_t*)W(ffn), (const uint16_t*)W(ffn + 1), (const uint16_t*)nullptr,
        (const uint16_t*)nullptr, (const int*)nullptr, (const float*)nullptr, (const float*)nullptr,
        0, 0, (int)d.I, 0, s->act);
      residual(L, s->act, W(ffn + 2), d.H, d.I, s->attn, s->h);
    }
    base += layer_tensors(c, l);
  }
  if (last) {
    const int64_t total = weight_count(c);
    project32<true>(L, KC_LOGITS, s->h, (const float*)Wt(total - 2), c.eps,
                    segments({{Wt(total - 1), {s->logits, d.V}}}), d.H, s->d_best);
  }
}

void enqueue_shadow(cq35_session* s, bool import) {
  const Dims& d = s->model->d;
  Launcher L{s};
  const int64_t base = s->capacity * d.KV_STRIDE;
  const int blocks = grid_for((d.L * d.REC + kBlock - 1) / kBlock, 8192);
  if (import)
    L(KC_SHADOW, k_import, dim3(blocks), dim3(kBlock), 0, (const uint16_t*)s->cache, base, d.LIN,
      d.CONV, d.REC, (int)d.L, s->shadow);
  else
    L(KC_SHADOW, k_persist, dim3(blocks), dim3(kBlock), 0, s->cache, base, d.LIN, d.CONV, d.REC,
      (int)d.L, (const float*)s->shadow);
}

// Shapes the batched prefill kernels accept (quad loads, scan width, the
// shared-expert lanes inside the routed loop); empty when supported.
const char* prefill_unsupported(const cq35_model& m) {
  const Dims& d = m.d;
  const cq35_config& c = m.cfg;
  if (d.H % 8 || d.QS % 8 || d.VS % 8) return "hidden, query and value widths must be multiples of 8";
  if (c.key_dim > 256) return "key_dim above 256";
  if (c.key_dim != 32 && c.key_dim != 64 && c.key_dim != 128 && c.key_dim != 256)
    return "key_dim must be 32, 64, 128 or 256";
  if (c.value_dim % 8) return "value_dim must be a multiple of 8 (eight channels of one head per scan block)";
  if (bscan_lds_bytes(c.key_dim) > 65536) return "key_dim too large for the scan's LDS stage";
  if (d.I % 8) return "intermediate width must be a multiple of 8";
  if (c.moe && (d.SI % 8 || d.SI > d.K * d.I))
    return "shared-expert width must be a multiple of 8 and at most top_k * intermediate";
  if (c.moe && d.K > 64) return "top_k above 64";
  return nullptr;
}

// Chunk buffers of the batched prefill: kBChunk token rows, or kMChunk when
// the session has matrix-core components selected at its first multi-token
// call (their expert weights are then streamed once per kMChunk tokens).
int setup_prefill(cq35_session* s) {
  if (s->pf_ready) return CQ35_OK;
  const Dims& d = s->model->d;
  const cq35_config& c = s->model->cfg;
  const int64_t m = s->matrix ? kMChunk : kBChunk, VH = c.value_heads;
  s->pf_rows = (int)m;
  int rc = CQ35_OK;
  auto check = [&](int r) { if (r && !rc) rc = r; };
  check(dalloc(s, &s->pf_h, m * d.H));
  check(dalloc(s, &s->pf_x, m * d.H));
  check(dalloc(s, &s->pf_attn, m * d.H));
  check(dalloc(s, &s->pf_a, m * std::max(d.QKV, 2 * d.QS)));  // qkv | qg
  check(dalloc(s, &s->pf_b, m * std::max(d.VS, d.KVS)));      // z | k
  check(dalloc(s, &s->pf_c, m * std::max(2 * VH, d.KVS)));    // alpha, beta | v
  check(dalloc(s, &s->pf_d, m * std::max(d.QKV, d.QS)));      // conv | rotated q
  check(dalloc(s, &s->pf_e, m * 2 * d.KS));                   // l2 q, k
  check(dalloc(s, &s->pf_f, m * std::max(d.VS, d.QS)));       // core | context
  check(dalloc(s, &s->pf_g, m * d.VS));                       // gated
  check(dalloc(s, &s->pf_act, m * std::max(d.I, d.K * d.I + d.SI)));
  check(dalloc(s, &s->pf_rope, m * std::max<int64_t>(d.R, 2)));
  if (c.moe) {
    check(dalloc(s, &s->pf_logits, m * (d.E + 1)));
    check(dalloc(s, &s->pf_ids, m * d.K));
    check(dalloc(s, &s->pf_probs, m * d.K));
    check(dalloc(s, &s->pf_eoff, d.E + 2));
    check(dalloc(s, &s->pf_order, m * d.K));
    check(dalloc(s, &s->pf_part, m * d.K * d.H));
    check(dalloc(s, &s->pf_spart, m * d.H));
  }
  // staged attention scratch rows, at most 64 MiB
  const int64_t per_token = d.Q * (int64_t)s->attn_stride;
  s->pf_attn_tokens = (int)std::max<int64_t>(1, std::min<int64_t>(m, (64ll << 20) / 4 / per_token));
  check(dalloc(s, &s->pf_scratch, s->pf_attn_tokens * per_token));
  if (rc) return rc;
  s->pf_ready = true;
  return CQ35_OK;
}

// The batched prefill of an n-token call (text-batch, prefill.rs:523-618):
// shadow import, then per chunk of kBChunk tokens the embedding rows and the
// layer fold over all rows (batch.full / batch.linear, prefill.rs:92-456),
// shadow persist, and the head on the call's last row (prefill.row).
void enqueue_prefill(cq35_session* s, int64_t n) {
  const cq35_model& m = *s->model;
  const cq35_config& c = m.cfg;
  const Dims& d = m.d;
  Launcher L{s};
  auto Wt = [&](int64_t index) { return m.w[index]; };
  const int64_t cap = s->capacity;
  const int H = (int)d.H, VH = c.value_heads;
  const uint64_t* params = s->d_params;
  enqueue_shadow(s, true);
  int last_rows = 1;
  // The chunk size changes no result (every per-token operation is
  // independent of the other rows, the scan carries its state in the shadow),
  // so the matrix-core components take larger chunks when the buffers allow.
  const int64_t chunk = s->matrix ? s->pf_rows : std::min<int64_t>(kBChunk, s->pf_rows);
  for (int64_t c0 = 0; c0 < n; c0 += chunk) {
    const int rows_n = (int)std::min<int64_t>(chunk, n - c0);
    const int first = (int)c0;
    const unsigned tiles = (unsigned)((rows_n + 4 * kBTokens - 1) / (4 * kBTokens));
    L(KC_EMBED, k_bembed, dim3(rows_n), dim3(kBlock), 0, params, first, (const uint16_t*)Wt(0), H,
      s->pf_h, c0 + rows_n == n ? s->d_best : (unsigned long long*)nullptr);
    // matrix-core projections when selected (K a multiple of the MFMA step)
    const bool mp = (s->matrix & CQ35_MATRIX_PROJECTIONS) != 0;
    // matrix-core projections: LDS-staged tiles for widths of whole 128-column
    // pairs of steps, the direct kernel (same order) for other multiples of 16
    const unsigned mtiles = (unsigned)((rows_n + kMBlockTokens - 1) / kMBlockTokens);
    auto staged = [&](int cols) { return cols % (2 * kGBK) == 0; };
    auto mgrid = [&](int rows, int cols) {
      return staged(cols) ? dim3((unsigned)gemm_grid(rows, rows_n))
                          : dim3((unsigned)((rows + kMRows - 1) / kMRows), mtiles);
    };
    // several projections of one input: one staged launch over their
    // concatenated rows, else one launch each
    auto project_all = [&](const uint16_t* x, int cols, const Segments& seg) {
      if (mp && staged(cols)) {
        L(KC_PREFILL_PROJECT, k_mgemm<kBPlain>, mgrid((int)seg_rows(seg), cols), dim3(64 * kMWaves), 0, x,
          rows_n, cols, seg, (const uint16_t*)nullptr, (const uint16_t*)nullptr);
        return true;
      }
      return false;
    };
    auto project = [&](const uint16_t* x, int cols, const void* w, int rows, uint16_t* out) {
      if (mp && staged(cols))
        L(KC_PREFILL_PROJECT, k_mgemm<kBPlain>, mgrid(rows, cols), dim3(64 * kMWaves), 0, x, rows_n, cols,
          segments({{w, {out, rows}}}), (const uint16_t*)nullptr, (const uint16_t*)nullptr);
      else if (mp && cols % 16 == 0)
        L(KC_PREFILL_PROJECT, k_mproject<kBPlain>, mgrid(rows, cols), dim3(64 * kMWaves), 0, x, rows_n, cols,
          (const uint16_t*)w, (const uint16_t*)nullptr, rows, (const uint16_t*)nullptr, out);
      else
        L(KC_PREFILL_PROJECT, k_bproject<kBPlain>,
          dim3((unsigned)((rows + bproject_rows<kBPlain>() - 1) / bproject_rows<kBPlain>()), tiles), dim3(kBlock), 0, x,
          rows_n, cols, (const uint16_t*)w, (const uint16_t*)nullptr, rows, (const uint16_t*)nullptr,
          out);
    };
    auto residual_rows = [&](const uint16_t* x, int cols, const void* w, const uint16_t* res,
                             uint16_t* out) {
      if (mp && staged(cols))
        L(KC_PREFILL_PROJECT, k_mgemm<kBResidual>, mgrid(H, cols), dim3(64 * kMWaves), 0, x, rows_n, cols,
          segments({{w, {out, H}}}), (const uint16_t*)nullptr, res);
      else if (mp && cols % 16 == 0)
        L(KC_PREFILL_PROJECT, k_mproject<kBResidual>, mgrid(H, cols), dim3(64 * kMWaves), 0, x, rows_n, cols,
          (const uint16_t*)w, (const uint16_t*)nullptr, H, res, out);
      else
        L(KC_PREFILL_PROJECT, k_bproject<kBResidual>,
          dim3((unsigned)((H + bproject_rows<kBResidual>() - 1) / bproject_rows<kBResidual>()), tiles), dim3(kBlock), 0, x,
          rows_n, cols, (const uint16_t*)w, (const uint16_t*)nullptr, H, res, out);
    };
    auto norm = [&](const uint16_t* x, const void* w, uint16_t* out) {
      L(KC_PROJECT, k_bnorm, dim3(rows_n), dim3(kBlock), (size_t)H * 2, x, (const float*)w, H,
        c.eps, out);
    };
    int64_t base = 1;
    for (int64_t l = 0; l < d.L; ++l) {
      auto W = [&](int slot) { return Wt(base + slot); };
      const int64_t key_base = l * 2 * cap * d.KVS;
      const int64_t value_base = key_base + cap * d.KVS;
      norm(s->pf_h, W(0), s->pf_x);
      int ffn;
      const void* post_norm;
      if (is_full(c, l)) {
        uint16_t *qg = s->pf_a, *kraw = s->pf_b, *vraw = s->pf_c, *qr = s->pf_d, *ctx = s->pf_f;
        if (!project_all(s->pf_x, H, segments({{W(1), {qg, 2 * d.QS}}, {W(2), {kraw, d.KVS}}, {W(3), {vraw, d.KVS}}}))) {
          project(s->pf_x, H, W(1), (int)(2 * d.QS), qg);
          project(s->pf_x, H, W(2), (int)d.KVS, kraw);
          project(s->pf_x, H, W(3), (int)d.KVS, vraw);
        }
        L(KC_EMBED, k_brope, dim3(rows_n), dim3(kBlock), 0, params, first, (const float*)m.freq,
          (int)(d.R / 2), s->pf_rope);
        L(KC_PREPARE_FULL, k_full_prepare, dim3((unsigned)(d.Q + d.KVH), rows_n), dim3(kBlock), 0,
          (const uint16_t*)qg, (const uint16_t*)kraw, (const uint16_t*)vraw,
          (const float*)s->pf_rope, (const float*)W(5), (const float*)W(6), s->cache, key_base,
          value_base, params, first, (int)d.KVS, (int)d.Q, (int)d.HD, d.pad_hd, (int)d.R, c.eps, qr, (const SessionRows*)nullptr);
        const float scale = 1.0f / sqrtf((float)d.HD);  // SCALE_BITS, qwen35.rs:701
        auto mattention = [&](auto kernel) {
          L(KC_ATTENTION, kernel, dim3((unsigned)d.Q, (unsigned)((rows_n + 31) / 32)), dim3(64 * kAWaves), 0,
            (const uint16_t*)qr, (const uint16_t*)qg, (const uint16_t*)s->cache, key_base, value_base, params,
            first, rows_n, (int)d.KVS, (int)d.Q, (int)(d.Q / d.KVH), scale, ctx);
        };
        const bool ma = (s->matrix & CQ35_MATRIX_ATTENTION) != 0;
        if (ma && d.HD == 256) mattention(k_mattention<256>);
        else if (ma && d.HD == 128) mattention(k_mattention<128>);
        else if (ma && d.HD == 64) mattention(k_mattention<64>);
        else {  // the exact staged kernels
          // regrouped as in the batched step (scores per key chunk and head
          // pair, the softmax, the context per KV head) where the shape
          // allows: the same chains and rounding
          const int hpk = (int)(d.Q / d.KVH);
          const bool regroup = d.HD % 8 == 0 && d.HD <= 256 && (hpk == 1 || hpk == 2 || hpk == 4 || hpk == 8);
          const int64_t start = (int64_t)s->h_params[0];  // the call's first position
          for (int a0 = 0; a0 < rows_n; a0 += s->pf_attn_tokens) {
            const int am = std::min(s->pf_attn_tokens, rows_n - a0);
            const uint16_t* qa = qr + (size_t)a0 * d.QS;
            if (regroup) {
              const unsigned chunks = (unsigned)((start + first + a0 + am + 255) / 256);  // keys of the last token
              if (hpk % 2 == 0)
                L(KC_ATTENTION, k_bstaged_scores<2>, dim3(chunks, (unsigned)(d.KVH * hpk / 2), (unsigned)am), dim3(256), 0,
                  qa, (const SessionRows*)nullptr, (const uint16_t*)s->cache, params, first + a0, key_base, (int)d.KVS,
                  (int)d.HD, (int)d.Q, hpk, scale, s->pf_scratch, s->attn_stride);
              else
                L(KC_ATTENTION, k_bstaged_scores<1>, dim3(chunks, (unsigned)(d.KVH * hpk), (unsigned)am), dim3(256), 0,
                  qa, (const SessionRows*)nullptr, (const uint16_t*)s->cache, params, first + a0, key_base, (int)d.KVS,
                  (int)d.HD, (int)d.Q, hpk, scale, s->pf_scratch, s->attn_stride);
            }
            L(KC_ATTENTION, k_attention_staged, dim3((unsigned)d.Q, (unsigned)am), dim3(kStagedThreads), 0,
              qa, (const uint16_t*)s->cache, key_base, params,
              first + a0, (int)d.KVS, (int)d.HD, hpk, scale, s->pf_scratch, s->attn_stride, (const SessionRows*)nullptr,
              regroup);
            const uint16_t* qga = qg + (size_t)a0 * 2 * d.QS;
            uint16_t* ca = ctx + (size_t)a0 * d.QS;
            const dim3 cgrid((unsigned)(d.KVH * d.HD / kContextChannels), (unsigned)am);
            auto grouped = [&](auto kernel) {
              L(KC_ATTENTION, kernel, cgrid, dim3(kContextThreads), 0, (const uint16_t*)s->cache, params, first + a0,
                value_base, (int)d.KVS, (int)d.HD, (int)d.Q, qga, (const float*)s->pf_scratch, s->attn_stride, ca,
                (const SessionRows*)nullptr);
            };
            if (regroup && hpk == 1) grouped(k_battention_context<1>);
            else if (regroup && hpk == 2) grouped(k_battention_context<2>);
            else if (regroup && hpk == 4) grouped(k_battention_context<4>);
            else if (regroup && hpk == 8) grouped(k_battention_context<8>);
            else
              L(KC_ATTENTION, k_attention_context, dim3((unsigned)(d.Q * d.HD / kContextChannels), (unsigned)am),
                dim3(kContextThreads), 0, (const uint16_t*)s->cache, value_base, params, first + a0, (int)d.KVS,
                (int)d.HD, (int)d.Q, hpk, qga, (const float*)s->pf_scratch, s->attn_stride, ca,
                (const SessionRows*)nullptr);
          }
        }
        residual_rows(ctx, (int)d.QS, W(4), s->pf_h, s->pf_attn);
        post_norm = W(7);
        ffn = 8;
      } else {
        uint16_t *qkv = s->pf_a, *z = s->pf_b, *alpha = s->pf_c, *beta = s->pf_c + (size_t)s->pf_rows * VH;
        uint16_t *conv = s->pf_d, *qn = s->pf_e, *kn = s->pf_e + (size_t)s->pf_rows * d.KS;
        uint16_t *core = s->pf_f, *gated = s->pf_g;
        if (!project_all(s->pf_x, H,
                         segments({{W(1), {qkv, d.QKV}}, {W(2), {z, d.VS}}, {W(3), {alpha, VH}}, {W(4), {beta, VH}}}))) {
          project(s->pf_x, H, W(1), (int)d.QKV, qkv);
          project(s->pf_x, H, W(2), (int)d.VS, z);
          project(s->pf_x, H, W(3), VH, alpha);
          project(s->pf_x, H, W(4), VH, beta);
        }
        const int64_t conv_base = cap * d.KV_STRIDE + l * d.LIN;
        L(KC_PREPARE_LINEAR, k_bprepare,
          dim3((unsigned)((d.QKV + c.key_dim - 1) / c.key_dim), rows_n), dim3(kBlock), 0,
          (const uint16_t*)qkv, (const uint16_t*)s->cache, conv_base, params, first,
          (const float*)W(9), (int)d.QKV, c.key_dim, c.key_heads, conv, qn, kn);
        L(KC_PREPARE_LINEAR, k_bhistory, dim3(grid_for((3 * d.QKV + kBlock - 1) / kBlock, 1024)),
          dim3(kBlock), 0, (const uint16_t*)qkv, rows_n, s->cache, conv_base, params, first,
          (int)d.QKV);
        const float scale = 1.0f / sqrtf((float)c.key_dim);  // DELTA_SCALE_BITS, qwen35.rs:703
        auto scan = k_bscan<4>;  // key elements per lane: key_dim / 32
        if (c.key_dim == 32) scan = k_bscan<1>;
        else if (c.key_dim == 64) scan = k_bscan<2>;
        else if (c.key_dim == 256) scan = k_bscan<8>;
        L(KC_DELTA, scan, dim3((unsigned)((d.VS + 7) / 8)), dim3(kBlock), bscan_lds_bytes(c.key_dim),
          (const uint16_t*)conv, (const uint16_t*)qn, (const uint16_t*)kn, (const uint16_t*)alpha,
          (const uint16_t*)beta, (const float*)W(5), (const float*)W(6), s->shadow + l * d.REC,
          rows_n, (int)d.VS, c.value_dim, VH, c.key_dim, c.key_heads, (int)d.QKV, scale, core);
        L(KC_GATED_NORM, k_gated_norm, dim3((unsigned)(VH * rows_n)), dim3(kBlock), 0,
          (const uint16_t*)core, (const uint16_t*)z, (const float*)W(7), c.value_dim, c.eps, gated);
        residual_rows(gated, (int)d.VS, W(8), s->pf_h, s->pf_attn);
        post_norm = W(10);
        ffn = 11;
      }
      norm(s->pf_attn, post_norm, s->pf_x);
      if (c.moe) {
        const int E = (int)d.E, K = (int)d.K, I = (int)d.I, SI = (int)d.SI;
        const dim3 rgrid((unsigned)((E + kRouterRows) / kRouterRows),
                         (unsigned)((rows_n + kRouterTokens - 1) / kRouterTokens));
        auto router = [&](auto kernel) {
          L(KC_ROUTER, kernel, rgrid, dim3(512), 0, (const uint16_t*)s->pf_x, rows_n, (const float*)W(ffn),
            (const float*)W(ffn + 4), E, s->pf_logits);
        };
        if (H == 2048) router(k_brouter_shared<32>);
        else if (H == 1024) router(k_brouter_shared<16>);
        else if (H == 512) router(k_brouter_shared<8>);
        else if (H == 256) router(k_brouter_shared<4>);
        else
          L(KC_ROUTER, k_brouter, dim3((unsigned)((E + 1 + 3) / 4), rows_n), dim3(kBlock), 0,
            (const uint16_t*)s->pf_x, H, (const float*)W(ffn), (const float*)W(ffn + 4), E,
            s->pf_logits);
        L(KC_ROUTER, k_bselect, dim3(rows_n), dim3(kBlock), (size_t)E * 4,
          (const float*)s->pf_logits, E, K, s->pf_ids, s->pf_probs,
          c0 + rows_n == n ? s->ids + l * d.K : (int*)nullptr);
        const int rows = K * I + SI;
        if ((s->matrix & CQ35_MATRIX_EXPERTS) && H % 16 == 0 && I % 16 == 0 && SI % 16 == 0) {
          const int A = rows_n * K;
          L(KC_ROUTER, k_moe_bucket, dim3(1), dim3(1024), (size_t)E * 2 * sizeof(int),
            (const int*)s->pf_ids, A, E, s->pf_eoff, s->pf_order);
          const unsigned mt = (unsigned)((rows_n + 31) / 32);  // token tiles of the busiest expert at most
          L(KC_MOE_GATE, k_mmoe_gate, dim3((unsigned)((std::max(I, SI) + kXRows - 1) / kXRows), (unsigned)(E + 1), mt),
            dim3(64 * kXWaves), 0, (const uint16_t*)s->pf_x, H, (const uint16_t*)W(ffn + 1),
            (const uint16_t*)W(ffn + 2), (const uint16_t*)W(ffn + 5), (const uint16_t*)W(ffn + 6),
            (const int*)s->pf_eoff, (const int*)s->pf_order, (const float*)s->pf_probs,
            (const float*)s->pf_logits, E, K, I, SI, rows_n, s->pf_act);
          L(KC_MOE_DOWN, k_mmoe_down, dim3((unsigned)((H + kXRows - 1) / kXRows), (unsigned)(E + 1), mt),
            dim3(64 * kXWaves), 0, (const uint16_t*)s->pf_act, (const uint16_t*)W(ffn + 3),
            (const uint16_t*)W(ffn + 7), (const int*)s->pf_eoff, (const int*)s->pf_order, E, K, I, SI, H,
            rows_n, s->pf_part, s->pf_spart);
          L(KC_MOE_DOWN, k_moe_combine, dim3((unsigned)((H + kBlock - 1) / kBlock), (unsigned)rows_n),
            dim3(kBlock), 0, (const float*)s->pf_part, (const float*)s->pf_spart,
            (const uint16_t*)s->pf_attn, H, K, s->pf_h);
        } else {
          if (H <= 2048) {
            // the gate/up rows read once per chunk: assignments bucketed by expert
            L(KC_ROUTER, k_moe_bucket, dim3(1), dim3(1024), (size_t)E * 2 * sizeof(int),
              (const int*)s->pf_ids, rows_n * K, E, s->pf_eoff, s->pf_order);
            auto grouped = [&](auto routed, auto shared) {
              L(KC_MOE_GATE, routed, dim3((unsigned)((I + kGRows - 1) / kGRows), (unsigned)E), dim3(kBlock), 0,
                (const uint16_t*)s->pf_x, H, (const uint16_t*)W(ffn + 1), (const uint16_t*)W(ffn + 2),
                (const int*)s->pf_eoff, (const int*)s->pf_order, (const float*)s->pf_probs,
                (const float*)s->pf_logits, E, K, I, SI, rows_n, s->pf_act);
              L(KC_MOE_GATE, shared,
                dim3((unsigned)((SI + kGRows - 1) / kGRows), (unsigned)((rows_n + kGSharedTokens - 1) / kGSharedTokens)),
                dim3(kBlock), 0, (const uint16_t*)s->pf_x, H, (const uint16_t*)W(ffn + 5),
                (const uint16_t*)W(ffn + 6), (const int*)s->pf_eoff, (const int*)s->pf_order,
                (const float*)s->pf_probs, (const float*)s->pf_logits, E, K, I, SI, rows_n, s->pf_act);
            };
            if (H > 1024) grouped(k_bmoe_gate_grouped<4, false>, k_bmoe_gate_grouped<4, true>);
            else if (H > 512) grouped(k_bmoe_gate_grouped<2, false>, k_bmoe_gate_grouped<2, true>);
            else grouped(k_bmoe_gate_grouped<1, false>, k_bmoe_gate_grouped<1, true>);
          } else {
            L(KC_MOE_GATE, k_bmoe_gate, dim3((unsigned)((rows + 3) / 4), rows_n), dim3(kBlock), 0,
              (const uint16_t*)s->pf_x, H, (const uint16_t*)W(ffn + 1), (const uint16_t*)W(ffn + 2),
              (const uint16_t*)W(ffn + 5), (const uint16_t*)W(ffn + 6), (const int*)s->pf_ids,
              (const float*)s->pf_probs, (const float*)s->pf_logits, E, K, I, SI, s->pf_act);
          }
          auto down_rows = [&](auto kernel) {
            L(KC_MOE_DOWN, kernel, dim3((unsigned)bmoe_down_rows_grid(H, rows_n)), dim3(kBlock), 0,
              (const uint16_t*)s->pf_act, (const uint16_t*)W(ffn + 3), (const uint16_t*)W(ffn + 7),
              (const int*)s->pf_ids, (const uint16_t*)s->pf_attn, H, K, I, SI, rows_n, s->pf_h);
          };
          const int dq = (K * I / 8 + 63) / 64;  // routed quads per lane
          if (dq <= 1) down_rows(k_bmoe_down_rows<1>);
          else if (dq <= 2) down_rows(k_bmoe_down_rows<2>);
          else if (dq <= 4) down_rows(k_bmoe_down_rows<4>);
          else if (dq <= 8) down_rows(k_bmoe_down_rows<8>);
          else
            L(KC_MOE_DOWN, k_bmoe_down, dim3((unsigned)bmoe_down_grid(H, rows_n)), dim3(kBlock), 0,
              (const uint16_t*)s->pf_act, (const uint16_t*)W(ffn + 3), (const uint16_t*)W(ffn + 7),
              (const int*)s->pf_ids, (const uint16_t*)s->pf_attn, H, K, I, SI, rows_n, s->pf_h);
        }
      } else {
        if (mp && H % 16 == 0)
          if (staged(H))
            L(KC_PREFILL_PROJECT, k_mgemm<kBGate>, mgrid((int)d.I, H), dim3(64 * kMWaves), 0,
              (const uint16_t*)s->pf_x, rows_n, H, segments({{W(ffn), {s->pf_act, d.I}}}),
              (const uint16_t*)W(ffn + 1), (const uint16_t*)nullptr);
          else
            L(KC_PREFILL_PROJECT, k_mproject<kBGate>, mgrid((int)d.I, H), dim3(64 * kMWaves), 0,
              (const uint16_t*)s->pf_x, rows_n, H, (const uint16_t*)W(ffn), (const uint16_t*)W(ffn + 1),
              (int)d.I, (const uint16_t*)nullptr, s->pf_act);
        else
          L(KC_PREFILL_PROJECT, k_bproject<kBGate>, dim3((unsigned)d.I, tiles), dim3(kBlock), 0,
            (const uint16_t*)s->pf_x, rows_n, H, (const uint16_t*)W(ffn), (const uint16_t*)W(ffn + 1),
            (int)d.I, (const uint16_t*)nullptr, s->pf_act);
        residual_rows(s->pf_act, (int)d.I, W(ffn + 2), s->pf_attn, s->pf_h);
      }
      base += layer_tensors(c, l);
    }
    last_rows = rows_n;
  }
  enqueue_shadow(s, false);
  const int64_t total = weight_count(c);
  project32<true>(L, KC_LOGITS, s->pf_h + (size_t)(last_rows - 1) * d.H, (const float*)Wt(total - 2),
                  c.eps, segments({{Wt(total - 1), {s->logits, d.V}}}), d.H, s->d_best);
}

uint64_t decode_key(unsigned long long key) {
  if (key == 0) return 0;
  return (uint64_t)(0xffffffffu - (uint32_t)(key & 0xffffffffull));
}

int collect_timing(cq35_session* s) {
  for (int i = 0; i < s->ev_used; ++i) {
    float ms = 0.0f;
    HIP_TRY(hipEventElapsedTime(&ms, s->ev[2 * i], s->ev[2 * i + 1]));
    s->timed_ms += ms;
    ++s->timed_launches;
  }
  s->ev_used = 0;
  return CQ35_OK;
}

}  // namespace

namespace {

// One decode step through the persistent kernel: upload (position, token,
// step tag), one launch, read back the argmax key and the kernel's error word.
// The persistent step needs every CU: its blocks wait on each other, so two
// of them sharing the device could each hold part of the CUs and stall until
// their spin limits. Steps of different sessions on one device therefore run
// one at a time, from launch to completion.
std::mutex& persistent_lock(int device) {
  static std::mutex locks[64];
  return locks[device & 63];
}

int step_persistent(cq35_session* s, uint64_t token, int64_t start, uint64_t* next_token,
                    uint16_t* logits) {
  std::lock_guard<std::mutex> hold(persistent_lock(s->model->device));
  const cq35_config& c = s->model->cfg;
  if (++s->seq == 0) s->seq = 1;  // tag 0 marks never-written words
  s->h_params[0] = (uint64_t)start;
  s->h_params[1] = token;
  s->h_params[2] = s->seq;
  s->poisoned = true;  // cleared on success
  hipError_t e = hipMemcpyAsync(s->d_params, s->h_params, 3 * sizeof(uint64_t), hipMemcpyHostToDevice,
                                s->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "parameter upload: %s", hipGetErrorString(e));
  const MegaArgs* args = s->d_margs;
  void* kargs[] = {(void*)&args};
  const bool timed = s->timed_class == KC_DECODE_STEP && s->ev_used < kMaxTimedEvents;
  if (s->mega_coop) {
    if (timed) e = hipEventRecord(s->ev[2 * s->ev_used], s->stream);
    if (e == hipSuccess)
      e = hipLaunchCooperativeKernel(s->mega_kernel, dim3((unsigned)s->mega_grid), dim3(kMT), kargs,
                                     (unsigned)s->mega_lds, s->stream);
    if (e == hipSuccess && timed) e = hipEventRecord(s->ev[2 * s->ev_used + 1], s->stream);
    if (timed) ++s->ev_used;
  } else if (timed) {
    // events stamped by the dispatch packet, as for the per-kernel classes
    e = hipExtLaunchKernel(s->mega_kernel, dim3((unsigned)s->mega_grid), dim3(kMT), kargs, (size_t)s->mega_lds,
                           s->stream, s->ev[2 * s->ev_used], s->ev[2 * s->ev_used + 1], 0);
    ++s->ev_used;
  } else {
    e = hipLaunchKernel(s->mega_kernel, dim3((unsigned)s->mega_grid), dim3(kMT), kargs, (size_t)s->mega_lds,
                        s->stream);
  }
  if (e == hipSuccess) e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(s->h_best, s->d_best, 2 * sizeof(unsigned long long), hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess && logits)
    e = hipMemcpyAsync(logits, s->logits, (size_t)c.vocab * 2, hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "persistent step: %s", hipGetErrorString(e));
  if (s->timed_class >= 0) {
    int rc = collect_timing(s);
    if (rc) return rc;
  }
  if ((uint32_t)s->h_best[1] == s->seq)  // the error word holds the tag of the step that raised it
    return fail(CQ35_EDEVICE, "persistent step: an exchange wait exceeded its spin limit");
  const uint64_t t = decode_key(s->h_best[0]);
  if (t >= (uint64_t)c.vocab)
    return fail(CQ35_EDEVICE, "qwen3 returned next-token ID %llu outside the vocabulary", (unsigned long long)t);
  *next_token = t;
  s->poisoned = false;
  return CQ35_OK;
}

}  // namespace

extern "C" int cq35_session_set_persistent(cq35_session* s, int enabled) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  if (enabled && !s->mega_ok)
    return fail(CQ35_EUNSUPPORTED, "this model shape or capacity is outside the persistent decode kernel");
  s->mega_on = enabled != 0;
  return CQ35_OK;
}

extern "C" int cq35_session_set_attention_split(cq35_session* s, int64_t keys) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  if (keys < 0) return fail(CQ35_EINVAL, "split threshold %lld is negative", (long long)keys);
  if (keys == s->split_keys) return CQ35_OK;
  HIP_TRY(hipSetDevice(s->model->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  s->split_keys = keys;
  // the captured decode graph and the persistent kernel's arguments hold it
  if (s->graph_exec) {
    hipGraphExecDestroy(s->graph_exec);
    s->graph_exec = nullptr;
  }
  if (s->graph) {
    hipGraphDestroy(s->graph);
    s->graph = nullptr;
  }
  if (s->mega_ok) {
    s->margs.split_keys = keys;
    HIP_TRY(hipMemcpy(s->d_margs, &s->margs, sizeof(MegaArgs), hipMemcpyHostToDevice));
  }
  return CQ35_OK;
}

extern "C" int cq35_session_attention_split(const cq35_session* s, int64_t* keys) {
  if (!s || !keys) return fail(CQ35_EINVAL, "null argument");
  *keys = s->split_keys;
  return CQ35_OK;
}

extern "C" int cq35_session_phase_trace(const cq35_session* s, uint64_t* dst, int64_t count, int64_t* slots,
                                        int64_t* blocks) {
  if (!s || !slots || !blocks) return fail(CQ35_EINVAL, "null argument");
#ifdef CQ35_PHASE_TRACE
  if (!s->mega_ok) return fail(CQ35_EUNSUPPORTED, "the session has no persistent decode step");
  *slots = kTraceSlots;
  *blocks = s->mega_grid;
  const int64_t need = (int64_t)s->mega_grid * kTraceSlots;
  if (!dst) return CQ35_OK;
  if (count != need) return fail(CQ35_EINVAL, "the trace has %lld stamps", (long long)need);
  HIP_TRY(hipSetDevice(s->model->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  HIP_TRY(hipMemcpy(dst, s->margs.trace, need * sizeof(uint64_t), hipMemcpyDeviceToHost));
  return CQ35_OK;
#else
  (void)dst;
  (void)count;
  *slots = 0;
  *blocks = 0;
  return fail(CQ35_EUNSUPPORTED, "phase stamps exist only in a library built with CQ35_PHASE_TRACE");
#endif
}

extern "C" int cq35_session_set_matrix_prefill(cq35_session* s, int components) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  if (components & ~(CQ35_MATRIX_PROJECTIONS | CQ35_MATRIX_EXPERTS | CQ35_MATRIX_ATTENTION))
    return fail(CQ35_EINVAL, "unknown matrix-core prefill components %d", components);
  s->matrix = components;
  return CQ35_OK;
}

extern "C" int cq35_session_matrix_prefill(const cq35_session* s, int* components) {
  if (!s || !components) return fail(CQ35_EINVAL, "null argument");
  *components = s->matrix;
  return CQ35_OK;
}

extern "C" int cq35_session_set_matrix_decode(cq35_session* s, int enabled) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  if (enabled != 0 && enabled != 1) return fail(CQ35_EINVAL, "matrix decode option must be 0 or 1, not %d", enabled);
  s->matrix_decode = enabled;
  return CQ35_OK;
}

extern "C" int cq35_session_matrix_decode(const cq35_session* s, int* enabled) {
  if (!s || !enabled) return fail(CQ35_EINVAL, "null argument");
  *enabled = s->matrix_decode;
  return CQ35_OK;
}

extern "C" int cq35_session_persistent(const cq35_session* s, int* enabled) {
  if (!s || !enabled) return fail(CQ35_EINVAL, "null argument");
  *enabled = s->mega_on ? 1 : 0;
  return CQ35_OK;
}

extern "C" int cq35_session_init(cq35_model* m, int64_t capacity, cq35_session** out) {
  if (!m || !out) return fail(CQ35_EINVAL, "null argument");
  if (capacity <= 0) return fail(CQ35_EINVAL, "cache capacity must be non-zero");
  if (capacity > 262144) return fail(CQ35_ERANGE, "cache capacity %lld exceeds the model maximum 262144", (long long)capacity);
  HIP_TRY(hipSetDevice(m->device));
  if (m->cfg.moe) {
    // The exact-order attention keeps every key's weight of a head in LDS.
    const size_t lds = attn_values_lds_bytes(capacity);
    if (lds > 65536 &&
        hipFuncSetAttribute((const void*)k_attn_values, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(CQ35_EUNSUPPORTED, "capacity %lld needs %zu bytes of LDS for exact-order attention",
                  (long long)capacity, lds);
    if (moe_down_lds_optin(m->d) != hipSuccess)
      return fail(CQ35_EUNSUPPORTED, "expert widths need more LDS than the device grants");
  }
  return create_session(m, capacity, out);
}

extern "C" int cq35_session_free(cq35_session* s) {
  destroy_session(s);
  return CQ35_OK;
}

namespace {

// Enqueue a validated call on the session's stream (parameter upload, the
// launches, the token and logits readback), without waiting for it.
int step_launch(cq35_session* s, const uint64_t* tokens, int64_t n, int64_t start, uint16_t* logits) {
  const cq35_config& c = s->model->cfg;
  const bool batched = n >= 2 && c.key_dim == 128;
  hipError_t e;
  s->h_params[0] = (uint64_t)start;
  for (int64_t i = 0; i < n; ++i) s->h_params[1 + i] = tokens[i];
  s->poisoned = true;  // cleared on success
  e = hipMemcpyAsync(s->d_params, s->h_params, (n + 1) * sizeof(uint64_t), hipMemcpyHostToDevice,
                     s->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "parameter upload: %s", hipGetErrorString(e));
  // Dense calls import the BF16 recurrent state into the F32 shadow and
  // persist it afterwards; MoE only for multi-token calls
  // (qwen35.rs:1536-1545, 1591-1610). A single-token call is identical with
  // the state kept in BF16, which the decode path does directly.
  const bool shadow = n >= 2;
  const bool use_graph = n == 1 && s->graph_enabled && s->timed_class < 0;
  if (use_graph) {
    if (!s->graph_exec) {
      e = hipStreamBeginCapture(s->stream, hipStreamCaptureModeThreadLocal);
      if (e != hipSuccess) return fail(CQ35_EDEVICE, "graph capture: %s", hipGetErrorString(e));
      enqueue_token(s, 0, true, false);
      hipGraph_t graph = nullptr;
      e = hipStreamEndCapture(s->stream, &graph);
      if (e == hipSuccess) e = hipGraphInstantiate(&s->graph_exec, graph, nullptr, nullptr, 0);
      if (e != hipSuccess) {
        if (graph) hipGraphDestroy(graph);
        return fail(CQ35_EDEVICE, "graph instantiate: %s", hipGetErrorString(e));
      }
      s->graph = graph;
    }
    e = hipGraphLaunch(s->graph_exec, s->stream);
    if (e != hipSuccess) return fail(CQ35_EDEVICE, "graph launch: %s", hipGetErrorString(e));
  } else if (batched) {
    enqueue_prefill(s, n);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(CQ35_EDEVICE, "kernel launch: %s", hipGetErrorString(e));
  } else {
    if (shadow) enqueue_shadow(s, true);
    for (int64_t t = 0; t < n; ++t) enqueue_token(s, (int)t, t == n - 1, shadow);
    if (shadow) enqueue_shadow(s, false);
    e = hipGetLastError();
    if (e != hipSuccess) return fail(CQ35_EDEVICE, "kernel launch: %s", hipGetErrorString(e));
  }
  e = hipMemcpyAsync(s->h_best, s->d_best, sizeof(unsigned long long), hipMemcpyDeviceToHost, s->stream);
  if (e == hipSuccess && logits)
    e = hipMemcpyAsync(logits, s->logits, (size_t)c.vocab * 2, hipMemcpyDeviceToHost, s->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "step: %s", hipGetErrorString(e));
  return CQ35_OK;
}

// Wait for a launched call and return its next token.
int step_complete(cq35_session* s, uint64_t* next_token) {
  const cq35_config& c = s->model->cfg;
  hipError_t e = hipStreamSynchronize(s->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "step: %s", hipGetErrorString(e));
  if (s->timed_class >= 0) {
    int rc = collect_timing(s);
    if (rc) return rc;
  }
  const uint64_t token = decode_key(*s->h_best);
  if (token >= (uint64_t)c.vocab)
    return fail(CQ35_EDEVICE, "qwen3 returned next-token ID %llu outside the vocabulary",
                (unsigned long long)token);
  *next_token = token;
  s->poisoned = false;
  return CQ35_OK;
}

}  // namespace

extern "C" int cq35_step(cq35_session* s, const uint64_t* tokens, int64_t n, int64_t start,
                         int64_t capacity, uint64_t* next_token, uint16_t* logits) {
  if (!s || !tokens || !next_token) return fail(CQ35_EINVAL, "null argument");
  if (s->poisoned) return fail(CQ35_EPOISONED, "session state unavailable after failed execution");
  const cq35_config& c = s->model->cfg;
  // Validation before any work (src/model.rs:267-281, 697-709).
  if (n <= 0) return fail(CQ35_EINVAL, "the token prefix must not be empty");
  if (capacity != s->capacity)
    return fail(CQ35_EINVAL, "capacity %lld does not match the session's %lld", (long long)capacity,
                (long long)s->capacity);
  if (start < 0 || start + n > capacity)
    return fail(CQ35_ERANGE, "token range %lld..%lld exceeds cache capacity %lld", (long long)start,
                (long long)(start + n), (long long)capacity);
  for (int64_t i = 0; i < n; ++i)
    if (tokens[i] >= (uint64_t)c.vocab)
      return fail(CQ35_ERANGE, "token prefix contains an ID outside the %d-token vocabulary", c.vocab);
  // Multi-token calls at key_dim 128 take the batched prefill
  // (text-dispatch, prefill.rs:623-652); smaller key dims fold token by token.
  const bool batched = n >= 2 && c.key_dim == 128;
  if (batched) {
    if (const char* why = prefill_unsupported(*s->model))
      return fail(CQ35_EUNSUPPORTED, "batched prefill: %s", why);
  }
  hipError_t e = hipSetDevice(s->model->device);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "hipSetDevice: %s", hipGetErrorString(e));
  if (batched) {
    const int rc = setup_prefill(s);
    if (rc) return rc;
  }
  if (n == 1 && s->mega_on && (s->timed_class < 0 || s->timed_class == KC_DECODE_STEP))
    return step_persistent(s, tokens[0], start, next_token, logits);
  const int rc = step_launch(s, tokens, n, start, logits);
  return rc ? rc : step_complete(s, next_token);
}

namespace {

// ------------------------------------------------ weight-shared batched step

// Buffers of the batched decode step for sessions of one capacity: every
// activation row for up to `max_b` sessions, the session table and the
// argmax keys, and a captured graph per batch size (the table is rewritten
// before each replay, so a graph serves any sessions of that count).
struct BatchWorkspace {
  int64_t capacity = 0;
  int max_b = 0;
  hipStream_t stream = nullptr;
  SessionRows* d_rows = nullptr;
  SessionRows* h_rows = nullptr;  // pinned
  unsigned long long* d_best = nullptr;
  unsigned long long* h_best = nullptr;  // pinned
  uint16_t *h = nullptr, *x = nullptr, *attn = nullptr, *qkv = nullptr, *conv = nullptr, *z = nullptr;
  uint16_t *ab = nullptr, *qn = nullptr, *kn = nullptr, *core = nullptr, *gated = nullptr;
  uint16_t *qg = nullptr, *kraw = nullptr, *vraw = nullptr, *qr = nullptr, *ctx = nullptr, *act = nullptr;
  uint16_t* logits = nullptr;
  float *rope = nullptr, *scratch = nullptr;
  int stride = 0;
  float2* gates = nullptr;       // per session and value head (decay, rate)
  f32x16_t* mx_part = nullptr;  // matrix-core products: partial tiles of split column ranges
  unsigned long long* mx_keys = nullptr;  // and the head's per-tile argmax keys [token tiles][32-row tiles][32]
  // MoE: router logits [B][E + 1], top-k ids and weights [B][K], expert
  // activations [B][K * I + SI], split-K range partials [B][Q][128][2 + HD]
  float* rlogits = nullptr;
  int* bids = nullptr;
  float* bprobs = nullptr;
  uint16_t* bact = nullptr;
  float* part = nullptr;
  int* ecount = nullptr;  // per layer: (token, slot) entries per expert, then the distinct-expert count
  int* elist = nullptr;   // per layer and expert: the entries (token << 8 | slot, routing weight bits)
  int* uexp = nullptr;    // per layer: the round's distinct selected experts
  hipGraph_t graph[2][kMaxSessions + 1] = {};      // [matrix-core products][sessions]
  hipGraphExec_t exec[2][kMaxSessions + 1] = {};
  std::vector<void*> allocs;
};

void destroy_batch(BatchWorkspace* b) {
  if (!b) return;
  if (b->stream) hipStreamSynchronize(b->stream);
  for (int k = 0; k < 2; ++k)
    for (int i = 0; i <= kMaxSessions; ++i) {
      if (b->exec[k][i]) hipGraphExecDestroy(b->exec[k][i]);
      if (b->graph[k][i]) hipGraphDestroy(b->graph[k][i]);
    }
  for (void* p : b->allocs) hipFree(p);
  if (b->h_rows) hipHostFree(b->h_rows);
  if (b->h_best) hipHostFree(b->h_best);
  if (b->stream) hipStreamDestroy(b->stream);
  delete b;
}

int batch_workspace(cq35_model* m, int64_t capacity, int count, BatchWorkspace** out) {
  BatchWorkspace* b = m->batch;
  if (b && b->capacity == capacity && b->max_b >= count) {
    *out = b;
    return CQ35_OK;
  }
  destroy_batch(b);
  m->batch = nullptr;
  b = new (std::nothrow) BatchWorkspace();
  if (!b) return fail(CQ35_EINVAL, "out of host memory");
  const Dims& d = m->d;
  const cq35_config& c = m->cfg;
  const int B = count <= 16 ? 16 : kMaxSessions;
  b->capacity = capacity;
  b->max_b = B;
  hipError_t e = hipStreamCreateWithFlags(&b->stream, hipStreamNonBlocking);
  auto alloc = [&](auto** p, int64_t n) {
    if (e != hipSuccess) return;
    void* q = nullptr;
    e = hipMalloc(&q, std::max<int64_t>(n, 1) * (int64_t)sizeof(**p));
    if (e == hipSuccess) {
      b->allocs.push_back(q);
      *p = static_cast<std::remove_reference_t<decltype(*p)>>(q);
    }
  };
  alloc(&b->d_rows, 1);
  alloc(&b->d_best, B);
  const int64_t wide = std::max({d.QKV, 2 * d.QS, d.VS, d.I, d.H});
  for (uint16_t** p : {&b->h, &b->x, &b->attn}) alloc(p, B * d.H);
  alloc(&b->qkv, B * d.QKV);
  alloc(&b->conv, B * d.QKV);
  alloc(&b->z, B * d.VS);
  alloc(&b->ab, 2 * B * (int64_t)c.value_heads);
  alloc(&b->qn, B * d.KS);
  alloc(&b->kn, B * d.KS);
  alloc(&b->core, B * d.VS);
  alloc(&b->gated, B * d.VS);
  alloc(&b->qg, B * 2 * d.QS);
  alloc(&b->kraw, B * d.KVS);
  alloc(&b->vraw, B * d.KVS);
  alloc(&b->qr, B * d.QS);
  alloc(&b->ctx, B * d.QS);
  alloc(&b->act, B * std::max<int64_t>(d.I, 1));
  alloc(&b->logits, B * d.V);
  alloc(&b->rope, B * std::max<int64_t>(d.R, 2));
  const int64_t tiles = (capacity + 7) / 8;
  b->stride = (int)std::max<int64_t>(tiles * 8 + 2 * tiles + 16, 3 * capacity + 16);
  alloc(&b->scratch, B * d.Q * (int64_t)b->stride);
  // partial tiles: kb x tiles < 1024 (split launches have < 128 tiles), each
  // up to two matrices x two 32-row halves x 64 lanes
  alloc(&b->mx_part, (int64_t)1024 * 2 * 2 * 64);
  alloc(&b->gates, B * (int64_t)c.value_heads);
  alloc(&b->mx_keys, ((B + 31) / 32) * ((d.V + 31) / 32 + 2) * 32);
  if (c.moe) {
    alloc(&b->rlogits, B * (d.E + 1));
    alloc(&b->bids, B * d.K);
    alloc(&b->bprobs, B * d.K);
    alloc(&b->bact, B * (d.K * d.I + d.SI));
    alloc(&b->part, (int64_t)B * d.Q * kSplitRanges * (2 + d.HD));
    alloc(&b->ecount, d.L * (d.E + 1));
    alloc(&b->elist, 2 * d.L * d.E * B * d.K);  // (token << 8 | slot, weight) pairs
    alloc(&b->uexp, d.L * std::min<int64_t>(d.E, B * d.K));
  }
  (void)wide;
  if (e == hipSuccess) e = hipHostMalloc((void**)&b->h_rows, sizeof(SessionRows), hipHostMallocDefault);
  if (e == hipSuccess) e = hipHostMalloc((void**)&b->h_best, B * sizeof(unsigned long long), hipHostMallocDefault);
  if (e != hipSuccess) {
    destroy_batch(b);
    return fail(CQ35_EDEVICE, "batch workspace: %s", hipGetErrorString(e));
  }
  m->batch = b;
  *out = b;
  return CQ35_OK;
}

// Matrix-core products of the batched step (k_mskinny) take widths that are
// multiples of 512. The vocabulary head runs two MFMA tiles per wave; launches
// with fewer than 128 row tiles split the columns over kb blocks (a power of
// two, at most 8) so that about 512 blocks stream.
bool skinny_ok(int64_t cols) { return cols % (16 * kSkSplit * 2 * kSkBatch) == 0; }
template <int kMode, int kT>
void skinny_launch(hipStream_t st, const BatchWorkspace* b, const uint16_t* x, int B, int64_t cols,
                   const Segments& seg, const uint16_t* w2, const uint16_t* res, unsigned long long* best) {
  const int64_t rows = seg_rows(seg), rt = (rows + 32 * kT - 1) / (32 * kT), tt = (B + 31) / 32;
  int kb = 1;
  if (rt * tt < 128)
    while (kb < 8 && rt * tt * kb < 512 && cols % (512 * kb * 2) == 0) kb *= 2;
  const dim3 grid((unsigned)rt, (unsigned)tt, (unsigned)kb);
  // the head's per-tile maxima go to the key buffer, then one block per token
  unsigned long long* keys = kMode == kSArgmax ? b->mx_keys : best;
  k_mskinny<kMode, kT><<<grid, dim3(64 * kSkSplit), 0, st>>>(x, B, (int)cols, seg, w2, res, keys, b->mx_part);
  if (kb > 1)
    k_mskinny_finish<kMode, kT><<<dim3(grid.x, grid.y), dim3(64), 0, st>>>(b->mx_part, kb, B, seg, res, keys);
  if (kMode == kSArgmax) k_argmax_tiles<<<dim3((unsigned)B), dim3(256), 0, st>>>(keys, (int)(rt * kT), B, best);
}
template <int kMode>
void skinny(hipStream_t st, const BatchWorkspace* b, const uint16_t* x, int B, int64_t cols, const Segments& seg,
            const uint16_t* w2, const uint16_t* res, unsigned long long* best) {
  // two tiles per wave for the vocabulary head only (other launches are far
  // narrower; instantiating the gate mode with two tiles would spill)
  if constexpr (kMode == kSArgmax) {
    if (seg_rows(seg) >= 32768) {
      skinny_launch<kMode, 2>(st, b, x, B, cols, seg, w2, res, best);
      return;
    }
  }
  skinny_launch<kMode, 1>(st, b, x, B, cols, seg, w2, res, best);
}

// Weight-shared GEMV launches (k_ws32 / k_ws64 / k_ws256_swiglu) over B
// tokens, or with mx the matrix-core products where the width allows.
void ws32(hipStream_t st, const uint16_t* x, int B, const Segments& seg, int64_t cols, unsigned long long* best,
          const BatchWorkspace* mx = nullptr) {
  if (mx && skinny_ok(cols)) {
    if (best) skinny<kSArgmax>(st, mx, x, B, cols, seg, nullptr, nullptr, best);
    else skinny<kBPlain>(st, mx, x, B, cols, seg, nullptr, nullptr, nullptr);
    return;
  }
  const int groups = (B + kBatchNB - 1) / kBatchNB;
  const int row_blocks = (int)((seg_rows(seg) + 31) / 32);
  const size_t lds = (size_t)kBatchNB * std::min<int64_t>(cols, kBatchChunk) * 4;
  const dim3 grid((unsigned)batch_grid(row_blocks, groups)), block(kBlock);
  if (best) k_ws32<true, 8><<<grid, block, lds, st>>>(x, B, groups, seg, (int)cols, best);
  else k_ws32<false, 8><<<grid, block, lds, st>>>(x, B, groups, seg, (int)cols, best);
}
void ws64(hipStream_t st, const uint16_t* x, int B, const void* w, int64_t rows, int64_t cols, const uint16_t* res,
          uint16_t* out, const BatchWorkspace* mx = nullptr) {
  if (mx && skinny_ok(cols)) {
    const Segments one = segments({{w, {out, rows}}});
    if (res) skinny<kBResidual>(st, mx, x, B, cols, one, nullptr, res, nullptr);
    else skinny<kBPlain>(st, mx, x, B, cols, one, nullptr, nullptr, nullptr);
    return;
  }
  // two tokens per block: more blocks in flight (the other token groups'
  // weight reads hit the XCD's L2)
  constexpr int nb = 2;
  const int groups = (B + nb - 1) / nb;
  const int row_blocks = (int)((rows + 15) / 16);
  const size_t lds = (size_t)nb * std::min<int64_t>(cols, kBatchChunk) * 4;
  k_ws64<8, nb><<<dim3((unsigned)batch_grid(row_blocks, groups)), dim3(kBlock), lds, st>>>(
      x, B, groups, static_cast<const uint16_t*>(w), (int)rows, (int)cols, res, out);
}

// The batched decode step's launch sequence (dense models): every layer of
// enqueue_token for B sessions, GEMVs weight-shared, per-session kernels with
// one grid row per session. mx: the products on MFMA (k_mskinny) where the
// width allows.
void enqueue_batch(cq35_model* m, BatchWorkspace* b, int B, bool mx) {
  const cq35_config& c = m->cfg;
  const Dims& d = m->d;
  hipStream_t st = b->stream;
  auto Wt = [&](int64_t index) { return m->w[index]; };
  const int64_t cap = b->capacity;
  const SessionRows* rows = b->d_rows;
  k_sembed<<<dim3((unsigned)grid_for((d.H + kBlock - 1) / kBlock, 64), (unsigned)B), dim3(kBlock), 0, st>>>(
      rows, (const uint16_t*)Wt(0), (int)d.H, b->h, (const float*)m->freq, (int)(d.R / 2), b->rope, b->d_best);
  auto norm = [&](const uint16_t* x, const void* w, uint16_t* out) {
    k_bnorm<<<dim3((unsigned)B), dim3(kBlock), (size_t)d.H * 2, st>>>(x, (const float*)w, (int)d.H, c.eps, out);
  };
  int64_t base = 1;
  for (int64_t l = 0; l < d.L; ++l) {
    auto W = [&](int slot) { return Wt(base + slot); };
    const int64_t key_base = l * 2 * cap * d.KVS;
    const int64_t value_base = key_base + cap * d.KVS;
    norm(b->h, W(0), b->x);
    int ffn;
    const void* post_norm;
    if (is_full(c, l)) {
      ws32(st, b->x, B, segments({{W(1), {b->qg, 2 * d.QS}}, {W(2), {b->kraw, d.KVS}}, {W(3), {b->vraw, d.KVS}}}),
           d.H, nullptr, mx ? b : nullptr);
      k_full_prepare<<<dim3((unsigned)(d.Q + d.KVH), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->qg, (const uint16_t*)b->kraw, (const uint16_t*)b->vraw, (const float*)b->rope,
          (const float*)W(5), (const float*)W(6), (uint16_t*)nullptr, key_base, value_base,
          (const uint64_t*)nullptr, 0, (int)d.KVS, (int)d.Q, (int)d.HD, d.pad_hd, (int)d.R, c.eps, b->qr, rows);
      const float scale = 1.0f / sqrtf((float)d.HD);  // SCALE_BITS, qwen35.rs:701
      // scores over (key chunk, head pair, session), then the softmax per
      // (head, session); one query head per thread when hpk is odd
      const int hpk = (int)(d.Q / d.KVH);
      const bool scored = d.HD % 8 == 0 && d.HD <= 256;
      if (scored) {
        const unsigned chunks = (unsigned)((cap + 255) / 256);
        if (hpk % 2 == 0)
          k_bstaged_scores<2><<<dim3(chunks, (unsigned)(d.KVH * hpk / 2), (unsigned)B), dim3(256), 0, st>>>(
              (const uint16_t*)b->qr, rows, nullptr, nullptr, 0, key_base, (int)d.KVS, (int)d.HD, (int)d.Q, hpk, scale,
              b->scratch, b->stride);
        else
          k_bstaged_scores<1><<<dim3(chunks, (unsigned)(d.KVH * hpk), (unsigned)B), dim3(256), 0, st>>>(
              (const uint16_t*)b->qr, rows, nullptr, nullptr, 0, key_base, (int)d.KVS, (int)d.HD, (int)d.Q, hpk, scale,
              b->scratch, b->stride);
      }
      k_attention_staged<<<dim3((unsigned)d.Q, (unsigned)B), dim3(kStagedThreads), 0, st>>>(
          (const uint16_t*)b->qr, (const uint16_t*)nullptr, key_base, (const uint64_t*)nullptr, 0, (int)d.KVS,
          (int)d.HD, hpk, scale, b->scratch, b->stride, rows, scored);
      // the context per (KV head, channel chunk, session): each value slice
      // staged once for the KV head's query heads
      const dim3 cgrid((unsigned)(d.KVH * d.HD / kContextChannels), (unsigned)B);
      switch (hpk) {
        case 1: k_battention_context<1><<<cgrid, dim3(kContextThreads), 0, st>>>(nullptr, nullptr, 0, value_base, (int)d.KVS, (int)d.HD, (int)d.Q, (const uint16_t*)b->qg, (const float*)b->scratch, b->stride, b->ctx, rows); break;
        case 2: k_battention_context<2><<<cgrid, dim3(kContextThreads), 0, st>>>(nullptr, nullptr, 0, value_base, (int)d.KVS, (int)d.HD, (int)d.Q, (const uint16_t*)b->qg, (const float*)b->scratch, b->stride, b->ctx, rows); break;
        case 4: k_battention_context<4><<<cgrid, dim3(kContextThreads), 0, st>>>(nullptr, nullptr, 0, value_base, (int)d.KVS, (int)d.HD, (int)d.Q, (const uint16_t*)b->qg, (const float*)b->scratch, b->stride, b->ctx, rows); break;
        case 8: k_battention_context<8><<<cgrid, dim3(kContextThreads), 0, st>>>(nullptr, nullptr, 0, value_base, (int)d.KVS, (int)d.HD, (int)d.Q, (const uint16_t*)b->qg, (const float*)b->scratch, b->stride, b->ctx, rows); break;
        default:
          k_attention_context<<<dim3((unsigned)(d.Q * d.HD / kContextChannels), (unsigned)B), dim3(kContextThreads), 0, st>>>(
              (const uint16_t*)nullptr, value_base, (const uint64_t*)nullptr, 0, (int)d.KVS, (int)d.HD, (int)d.Q,
              hpk, (const uint16_t*)b->qg, (const float*)b->scratch, b->stride, b->ctx, rows);
      }
      ws64(st, b->ctx, B, W(4), d.H, d.QS, b->h, b->attn, mx ? b : nullptr);
      post_norm = W(7);
      ffn = 8;
    } else {
      uint16_t* alpha = b->ab;
      uint16_t* beta = b->ab + (size_t)B * c.value_heads;
      ws32(st, b->x, B,
           segments({{W(1), {b->qkv, d.QKV}}, {W(2), {b->z, d.VS}}, {W(3), {alpha, c.value_heads}},
                     {W(4), {beta, c.value_heads}}}),
           d.H, nullptr, mx ? b : nullptr);
      const int64_t conv_base = cap * d.KV_STRIDE + l * d.LIN;
      k_linear_prepare<<<dim3((unsigned)((d.QKV + c.key_dim - 1) / c.key_dim), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->qkv, (uint16_t*)nullptr, conv_base, (const uint64_t*)nullptr, 0, (const float*)W(9),
          (int)d.QKV, c.key_dim, c.key_heads, b->conv, b->qn, b->kn, rows, (const uint16_t*)alpha,
          (const uint16_t*)beta, (const float*)W(5), (const float*)W(6), c.value_heads, b->gates);
      const float scale = 1.0f / sqrtf((float)c.key_dim);  // DELTA_SCALE_BITS, qwen35.rs:703
      (c.key_dim == 128 ? k_delta<false, 128> : k_delta<false, 0>)<<<
          dim3((unsigned)((d.VS + 8 * kDeltaCh - 1) / (8 * kDeltaCh)), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->conv, (const uint16_t*)b->qn, (const uint16_t*)b->kn, (const float2*)b->gates,
          (uint16_t*)nullptr, (float*)nullptr,
          (int)d.VS, c.value_dim, c.key_dim, c.key_heads, (int)d.KS, scale, b->core, rows, conv_base + d.CONV);
      k_gated_norm<<<dim3((unsigned)c.value_heads, (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->core, (const uint16_t*)b->z, (const float*)W(7), c.value_dim, c.eps, b->gated);
      ws64(st, b->gated, B, W(8), d.H, d.VS, b->h, b->attn, mx ? b : nullptr);
      post_norm = W(10);
      ffn = 11;
    }
    norm(b->attn, post_norm, b->x);
    if (mx && skinny_ok(d.H)) {
      skinny<kBGate>(st, b, b->x, B, d.H, segments({{W(ffn), {b->act, d.I}}}), (const uint16_t*)W(ffn + 1), nullptr,
                     nullptr);
    } else {
      // two tokens per block (as the S64 products): more blocks in flight
      constexpr int nb = kBatchNBDual;
      const int groups = (B + nb - 1) / nb;
      const int row_blocks = (int)((d.I + 4 * kRowsGate - 1) / (4 * kRowsGate));
      k_ws256_swiglu<nb><<<dim3((unsigned)batch_grid(row_blocks, groups)), dim3(kBlock), (size_t)nb * d.H * 4, st>>>(
          b->x, B, groups, (const uint16_t*)W(ffn), (const uint16_t*)W(ffn + 1), (int)d.I, (int)d.H, b->act);
    }
    ws64(st, b->act, B, W(ffn + 2), d.H, d.I, b->attn, b->h, mx ? b : nullptr);
    base += layer_tensors(c, l);
  }
  const int64_t total = weight_count(c);
  norm(b->h, Wt(total - 2), b->x);
  ws32(st, b->x, B, segments({{Wt(total - 1), {b->logits, d.V}}}), d.H, b->d_best, mx ? b : nullptr);
}

// The batched decode step's launch sequence for MoE models: every layer of
// enqueue_token for B sessions, the non-expert products weight-shared (S256
// projections, S64 output projections, the router, the head), the routed
// experts once per distinct expert of the round, attention per session (split
// ranges or the single chain, each session's own threshold).
void enqueue_batch_moe(cq35_model* m, BatchWorkspace* b, int B) {
  const cq35_config& c = m->cfg;
  const Dims& d = m->d;
  hipStream_t st = b->stream;
  auto Wt = [&](int64_t index) { return m->w[index]; };
  const int64_t cap = b->capacity;
  const SessionRows* rows = b->d_rows;
  const int H = (int)d.H, E = (int)d.E, K = (int)d.K, I = (int)d.I, SI = (int)d.SI;
  const int groups = (B + kBatchNB - 1) / kBatchNB;
  k_sembed<<<dim3((unsigned)grid_for((d.H + kBlock - 1) / kBlock, 64), (unsigned)B), dim3(kBlock), 0, st>>>(
      rows, (const uint16_t*)Wt(0), H, b->h, (const float*)m->freq, (int)(d.R / 2), b->rope, b->d_best);
  const int max_b = b->max_b;
  const int max_slots = (int)std::min<int64_t>(d.E, (int64_t)max_b * d.K);
  k_zero_ints<<<dim3((unsigned)((d.L * (E + 1) + kBlock - 1) / kBlock)), dim3(kBlock), 0, st>>>(b->ecount,
                                                                                               (int)(d.L * (E + 1)));
  auto norm = [&](const uint16_t* x, const void* w, uint16_t* out) {
    k_bnorm<<<dim3((unsigned)B), dim3(kBlock), (size_t)d.H * 2, st>>>(x, (const float*)w, H, c.eps, out);
  };
  auto ws256 = [&](const uint16_t* x, const Segments& seg) {
    // two rows per wave; two tokens per block up to 8 sessions (more blocks
    // in flight, the other token groups' weight reads hit the XCD's L2),
    // four above
    const int row_blocks = (int)((seg_rows(seg) + 4 * 2 - 1) / (4 * 2));
    if (B <= 8)
      k_ws256<2, 2><<<dim3((unsigned)batch_grid(row_blocks, (B + 1) / 2)), dim3(kBlock), (size_t)2 * d.H * 4, st>>>(
          x, B, (B + 1) / 2, seg, H);
    else
      k_ws256<2, 4><<<dim3((unsigned)batch_grid(row_blocks, (B + 3) / 4)), dim3(kBlock), (size_t)4 * d.H * 4, st>>>(
          x, B, (B + 3) / 4, seg, H);
  };
  const int gate_blocks = (int)((std::max(d.I, d.SI) + kGateRowsPerBlock - 1) / kGateRowsPerBlock);
  const int hpk = (int)(d.Q / d.KVH);
  const int per_row = (int)((d.K * d.I + d.SI) / 8);
  int64_t base = 1;
  for (int64_t l = 0; l < d.L; ++l) {
    auto W = [&](int slot) { return Wt(base + slot); };
    const int64_t key_base = l * 2 * cap * d.KVS;
    const int64_t value_base = key_base + cap * d.KVS;
    norm(b->h, W(0), b->x);
    int ffn;
    const void* post_norm;
    if (is_full(c, l)) {
      ws256(b->x, segments({{W(1), {b->qg, 2 * d.QS}}, {W(2), {b->kraw, d.KVS}}, {W(3), {b->vraw, d.KVS}}}));
      k_full_prepare<<<dim3((unsigned)(d.Q + d.KVH), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->qg, (const uint16_t*)b->kraw, (const uint16_t*)b->vraw, (const float*)b->rope,
          (const float*)W(5), (const float*)W(6), (uint16_t*)nullptr, key_base, value_base,
          (const uint64_t*)nullptr, 0, (int)d.KVS, (int)d.Q, (int)d.HD, d.pad_hd, (int)d.R, c.eps, b->qr, rows);
      const float scale = 1.0f / sqrtf((float)d.HD);  // SCALE_BITS, qwen35.rs:701
      {
        // 16 keys per block per pass; about 2048 blocks over the batch
        const int per = (int)std::max<int64_t>(1, std::min<int64_t>((cap + 15) / 16, 2048 / (d.KVH * B)));
        const dim3 sg((unsigned)per, (unsigned)d.KVH, (unsigned)B);
        const uint16_t* qr = b->qr;
        if (hpk == 8 && d.HD == 256)
          k_bscores<8, 8><<<sg, dim3(kBlock), 0, st>>>(qr, rows, key_base, (int)d.KVS, scale, b->scratch, b->stride);
        else if (hpk == 2 && d.HD == 256)
          k_bscores<2, 8><<<sg, dim3(kBlock), 0, st>>>(qr, rows, key_base, (int)d.KVS, scale, b->scratch, b->stride);
        else if (hpk == 4 && d.HD == 64)
          k_bscores<4, 2><<<sg, dim3(kBlock), 0, st>>>(qr, rows, key_base, (int)d.KVS, scale, b->scratch, b->stride);
        else
          k_attn_scores<<<dim3((unsigned)std::min<int64_t>((cap + 7) / 8, 512), (unsigned)d.KVH, (unsigned)B),
                          dim3(kScoreBlock), (size_t)hpk * d.HD * 4, st>>>(
              qr, (const uint16_t*)nullptr, key_base, (const uint64_t*)nullptr, 0, (int)d.KVS, (int)d.HD, hpk, scale,
              b->scratch, b->stride, rows);
      }
      const dim3 fb((unsigned)flash_threads((int)d.HD));
      {
        const dim3 sgrid((unsigned)kSplitRanges, (unsigned)d.KVH, (unsigned)B);
        const float* sc = b->scratch;
        const uint16_t* qg = b->qg;
        const int KVS = (int)d.KVS, HD = (int)d.HD, Q = (int)d.Q;
        switch (hpk) {
          case 1: k_bflash<true, 1><<<sgrid, fb, 0, st>>>(sc, b->stride, rows, value_base, KVS, HD, Q, hpk, qg, b->part, b->ctx); break;
          case 2: k_bflash<true, 2><<<sgrid, fb, 0, st>>>(sc, b->stride, rows, value_base, KVS, HD, Q, hpk, qg, b->part, b->ctx); break;
          case 4: k_bflash<true, 4><<<sgrid, fb, 0, st>>>(sc, b->stride, rows, value_base, KVS, HD, Q, hpk, qg, b->part, b->ctx); break;
          default: k_bflash<true, 8><<<sgrid, fb, 0, st>>>(sc, b->stride, rows, value_base, KVS, HD, Q, hpk, qg, b->part, b->ctx); break;
        }
        k_bflash<false, 1><<<dim3(1u, (unsigned)d.Q, (unsigned)B), fb, 0, st>>>(sc, b->stride, rows, value_base, KVS,
                                                                                 HD, Q, hpk, qg, b->part, b->ctx);
      }
      k_bmerge<<<dim3((unsigned)d.Q, (unsigned)B), dim3(256), 0, st>>>((const float*)b->part, rows, (int)d.HD,
                                                                      (int)d.Q, (const uint16_t*)b->qg, b->ctx);
      ws64(st, b->ctx, B, W(4), d.H, d.QS, b->h, b->attn, nullptr);
      post_norm = W(7);
      ffn = 8;
    } else {
      uint16_t* alpha = b->ab;
      uint16_t* beta = b->ab + (size_t)B * c.value_heads;
      ws256(b->x, segments({{W(1), {b->qkv, d.QKV}}, {W(2), {b->z, d.VS}}, {W(3), {alpha, c.value_heads}},
                            {W(4), {beta, c.value_heads}}}));
      const int64_t conv_base = cap * d.KV_STRIDE + l * d.LIN;
      k_linear_prepare<<<dim3((unsigned)((d.QKV + c.key_dim - 1) / c.key_dim), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->qkv, (uint16_t*)nullptr, conv_base, (const uint64_t*)nullptr, 0, (const float*)W(9),
          (int)d.QKV, c.key_dim, c.key_heads, b->conv, b->qn, b->kn, rows, (const uint16_t*)alpha,
          (const uint16_t*)beta, (const float*)W(5), (const float*)W(6), c.value_heads, b->gates);
      const float scale = 1.0f / sqrtf((float)c.key_dim);  // DELTA_SCALE_BITS, qwen35.rs:703
      (c.key_dim == 128 ? k_delta<false, 128> : k_delta<false, 0>)<<<
          dim3((unsigned)((d.VS + 8 * kDeltaCh - 1) / (8 * kDeltaCh)), (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->conv, (const uint16_t*)b->qn, (const uint16_t*)b->kn, (const float2*)b->gates,
          (uint16_t*)nullptr, (float*)nullptr,
          (int)d.VS, c.value_dim, c.key_dim, c.key_heads, (int)d.KS, scale, b->core, rows, conv_base + d.CONV);
      k_gated_norm<<<dim3((unsigned)c.value_heads, (unsigned)B), dim3(kBlock), 0, st>>>(
          (const uint16_t*)b->core, (const uint16_t*)b->z, (const float*)W(7), c.value_dim, c.eps, b->gated);
      ws64(st, b->gated, B, W(8), d.H, d.VS, b->h, b->attn, nullptr);
      post_norm = W(10);
      ffn = 11;
    }
    {
      const dim3 rg((unsigned)((E + 1 + 3) / 4));
      const size_t rl = (size_t)B * d.H * 2;
      const float *pn = (const float*)post_norm, *rw = (const float*)W(ffn), *srw = (const float*)W(ffn + 4);
      switch (H) {
        case 2048: k_broute<32><<<rg, dim3(kBlock), rl, st>>>(b->attn, pn, c.eps, B, rw, srw, E, b->x, b->rlogits); break;
        case 1024: k_broute<16><<<rg, dim3(kBlock), rl, st>>>(b->attn, pn, c.eps, B, rw, srw, E, b->x, b->rlogits); break;
        case 512: k_broute<8><<<rg, dim3(kBlock), rl, st>>>(b->attn, pn, c.eps, B, rw, srw, E, b->x, b->rlogits); break;
        default: k_broute<4><<<rg, dim3(kBlock), rl, st>>>(b->attn, pn, c.eps, B, rw, srw, E, b->x, b->rlogits); break;
      }
    }
    int* ecount = b->ecount + l * (E + 1);
    int* elist = b->elist + 2 * l * E * max_b * K;
    int* uexp = b->uexp + l * max_slots;
    k_sselect<<<dim3((unsigned)((B + 3) / 4)), dim3(kBlock), (size_t)4 * E * 4, st>>>(
        b->rlogits, B, E, K, b->bids, b->bprobs, rows, (int)l, ecount, elist, max_b, uexp);
    {
      auto gate_kernel = H == 2048   ? k_bgate<4, true>
                         : H == 1024 ? k_bgate<2, true>
                         : H == 512  ? k_bgate<1, true>
                                     : k_bgate<1, false>;
      gate_kernel<<<dim3((unsigned)((max_slots + 1) * gate_blocks)), dim3(kBlock), 0, st>>>(
          b->x, B, H, (const uint16_t*)W(ffn + 1), (const uint16_t*)W(ffn + 2), (const uint16_t*)W(ffn + 5),
          (const uint16_t*)W(ffn + 6), ecount, elist, uexp, b->bprobs, b->rlogits, E, K, I, SI, gate_blocks,
          max_slots, max_b, b->bact);
    }
    k_bdown<<<dim3((unsigned)((d.H + kBDownRows - 1) / kBDownRows), (unsigned)((B + kBDownTokens - 1) / kBDownTokens)),
              dim3(kBlock), bdown_lds_bytes(per_row), st>>>(b->bact, B, (const uint16_t*)W(ffn + 3),
                                                             (const uint16_t*)W(ffn + 7), b->bids, b->attn, H, K, I, SI,
                                                             b->h);
    base += layer_tensors(c, l);
  }
  const int64_t total = weight_count(c);
  norm(b->h, Wt(total - 2), b->x);
  ws32(st, b->x, B, segments({{Wt(total - 1), {b->logits, d.V}}}), d.H, b->d_best, nullptr);
}

// One weight-shared decode step for `count` sessions of one model and
// capacity (checked by the caller): tokens[i] at starts[i] of sessions[i].
int step_batch_shared(cq35_session* const* sessions, const uint64_t* tokens, const int64_t* starts, int count,
                      uint64_t* next_tokens, uint16_t* logits) {
  cq35_model* m = sessions[0]->model;
  std::lock_guard<std::mutex> hold(m->batch_lock);
  HIP_TRY(hipSetDevice(m->device));
  BatchWorkspace* b = nullptr;
  int rc = batch_workspace(m, sessions[0]->capacity, count, &b);
  if (rc) return rc;
  const bool moe = m->cfg.moe != 0;
  for (int i = 0; i < count; ++i) {
    b->h_rows->cache[i] = sessions[i]->cache;
    b->h_rows->position[i] = (uint64_t)starts[i];
    b->h_rows->token[i] = tokens[i];
    b->h_rows->ids[i] = moe ? sessions[i]->ids : nullptr;
    b->h_rows->split[i] = sessions[i]->split_keys;
    sessions[i]->poisoned = true;  // cleared on success
  }
  // the products of dense models run on MFMA when every session selects
  // matrix-core decode (the MoE step has exact products only)
  bool mx = !moe;
  for (int i = 0; i < count; ++i) mx = mx && sessions[i]->matrix_decode != 0;
  hipError_t e = hipSuccess;
  for (int i = 0; i < count && e == hipSuccess; ++i) e = hipStreamSynchronize(sessions[i]->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(b->d_rows, b->h_rows, sizeof(SessionRows), hipMemcpyHostToDevice, b->stream);
  // CQ35_GRAPH=0 (as for sessions) enqueues the launches directly instead
  // of replaying a captured graph, e.g. for kernel tracing
  const char* graph_env = getenv("CQ35_GRAPH");
  const bool use_graph = !(graph_env && atoi(graph_env) == 0);
  auto enqueue = [&]() {
    if (moe) enqueue_batch_moe(m, b, count);
    else enqueue_batch(m, b, count, mx);
  };
  if (e == hipSuccess && !use_graph) enqueue();
  if (e == hipSuccess && use_graph && !b->exec[mx][count]) {
    e = hipStreamBeginCapture(b->stream, hipStreamCaptureModeThreadLocal);
    if (e == hipSuccess) {
      enqueue();
      hipGraph_t g = nullptr;
      e = hipStreamEndCapture(b->stream, &g);
      if (e == hipSuccess) e = hipGraphInstantiate(&b->exec[mx][count], g, nullptr, nullptr, 0);
      b->graph[mx][count] = g;
    }
  }
  if (e == hipSuccess && use_graph) e = hipGraphLaunch(b->exec[mx][count], b->stream);
  if (e == hipSuccess && !use_graph) e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(b->h_best, b->d_best, count * sizeof(unsigned long long), hipMemcpyDeviceToHost, b->stream);
  if (e == hipSuccess && logits)
    e = hipMemcpyAsync(logits, b->logits, (size_t)count * m->cfg.vocab * 2, hipMemcpyDeviceToHost, b->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(b->stream);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "batched step: %s", hipGetErrorString(e));
  for (int i = 0; i < count; ++i) {
    const uint64_t t = decode_key(b->h_best[i]);
    if (t >= (uint64_t)m->cfg.vocab)
      return fail(CQ35_EDEVICE, "qwen3 returned next-token ID %llu outside the vocabulary", (unsigned long long)t);
    next_tokens[i] = t;
  }
  for (int i = 0; i < count; ++i) sessions[i]->poisoned = false;
  return CQ35_OK;
}

// Whether the MoE shape fits the batched MoE kernels: a hidden width the
// router is instantiated for (staged once by k_ws256 and k_broute), expert
// and shared-expert widths in whole 64-element lane rounds of at most 512
// (k_bdown), the head dim within one flash block, 1, 2, 4 or 8 query heads
// per KV head and at most 16 experts selected per token.
bool moe_batch_shape_ok(const cq35_model* m) {
  const Dims& d = m->d;
  return (d.H == 2048 || d.H == 1024 || d.H == 512 || d.H == 256) && d.I % 64 == 0 && d.I <= 512 && d.E <= 512 && d.SI % 64 == 0 && d.SI <= 512 && d.HD <= 256 &&
         (d.Q / d.KVH == 1 || d.Q / d.KVH == 2 || d.Q / d.KVH == 4 || d.Q / d.KVH == 8) && d.K <= 16 && d.E <= 4096;
}

// Whether a batch can take the weight-shared step: sessions of one model and
// capacity, none of them timing kernels.
bool shared_batch_ok(cq35_session* const* sessions, int64_t count) {
  if (count < 2 || count > kMaxSessions) return false;
  if (const char* g = getenv("CQ35_BATCH_SHARED"))
    if (atoi(g) == 0) return false;
  const cq35_model* m = sessions[0]->model;
  if (m->cfg.hidden > kBatchChunk) return false;  // the SwiGLU and the S256 stage one row chunk
  if (m->cfg.moe && !moe_batch_shape_ok(m)) return false;
  // the MoE router stages every token's normalised row in LDS (64 KiB)
  if (m->cfg.moe && count * m->cfg.hidden * 2 > 65536) return false;
  for (int64_t i = 0; i < count; ++i)
    if (sessions[i]->model != m || sessions[i]->capacity != sessions[0]->capacity || sessions[i]->timed_class >= 0)
      return false;
  return true;
}

}  // namespace

extern "C" int cq35_step_batch(cq35_session* const* sessions, const uint64_t* tokens,
                               const int64_t* starts, int64_t count, uint64_t* next_tokens, uint16_t* logits) {
  if (!sessions || !tokens || !starts || !next_tokens || count <= 0) return fail(CQ35_EINVAL, "null argument");
  // every check before any work, as for one session
  for (int64_t i = 0; i < count; ++i) {
    cq35_session* s = sessions[i];
    if (!s) return fail(CQ35_EINVAL, "session %lld is null", (long long)i);
    if (s->poisoned) return fail(CQ35_EPOISONED, "session %lld state unavailable after failed execution", (long long)i);
    for (int64_t j = 0; j < i; ++j)
      if (sessions[j] == s) return fail(CQ35_EINVAL, "session %lld appears twice in the batch", (long long)i);
    if (starts[i] < 0 || starts[i] + 1 > s->capacity)
      return fail(CQ35_ERANGE, "session %lld: position %lld exceeds cache capacity %lld", (long long)i,
                  (long long)starts[i], (long long)s->capacity);
    if (tokens[i] >= (uint64_t)s->model->cfg.vocab)
      return fail(CQ35_ERANGE, "session %lld: token ID outside the %d-token vocabulary", (long long)i,
                  s->model->cfg.vocab);
  }
  if (shared_batch_ok(sessions, count)) {
    const int rc = step_batch_shared(sessions, tokens, starts, (int)count, next_tokens, logits);
    if (rc)
      for (int64_t i = 0; i < count; ++i) sessions[i]->poisoned = true;
    return rc;
  }
  // per-kernel sessions: launch all, then complete all (they overlap on the
  // device); persistent sessions step one at a time (each needs every CU)
  std::vector<int64_t> launched;
  for (int64_t i = 0; i < count; ++i) {
    cq35_session* s = sessions[i];
    HIP_TRY(hipSetDevice(s->model->device));
    int rc;
    uint16_t* li = logits ? logits + (size_t)i * s->model->cfg.vocab : nullptr;
    if (s->mega_on && s->timed_class < 0) {
      rc = step_persistent(s, tokens[i], starts[i], &next_tokens[i], li);
    } else {
      rc = step_launch(s, &tokens[i], 1, starts[i], li);
      if (!rc) launched.push_back(i);
    }
    if (rc) {
      // Sessions stepped or launched before the failure have moved, and the
      // caller cannot tell which: all of them become unusable, as the
      // failing one is (the caller restores them from checkpoints).
      for (int64_t j : launched) {
        uint64_t unused;
        step_complete(sessions[j], &unused);  // let the launched work finish
      }
      for (int64_t j = 0; j <= i; ++j) sessions[j]->poisoned = true;
      return rc;
    }
  }
  int first_error = CQ35_OK;
  for (int64_t i : launched) {
    const int rc = step_complete(sessions[i], &next_tokens[i]);
    if (rc && !first_error) first_error = rc;
  }
  if (first_error)
    for (int64_t i = 0; i < count; ++i) sessions[i]->poisoned = true;
  return first_error;
}

extern "C" int cq35_session_copy(const cq35_session* src, cq35_session** out) {
  if (!src || !out) return fail(CQ35_EINVAL, "null argument");
  if (src->poisoned) return fail(CQ35_EPOISONED, "session state unavailable after failed execution");
  HIP_TRY(hipSetDevice(src->model->device));
  cq35_session* s = nullptr;
  int rc = create_session(src->model, src->capacity, &s);
  if (rc) return rc;
  const Dims& d = src->model->d;
  hipError_t e = hipMemcpy(s->cache, src->cache, cache_elements(src->model->cfg, src->capacity) * 2,
                           hipMemcpyDeviceToDevice);
  if (e == hipSuccess) e = hipMemcpy(s->shadow, src->shadow, d.L * d.REC * 4, hipMemcpyDeviceToDevice);
  if (e != hipSuccess) {
    destroy_session(s);
    return fail(CQ35_EDEVICE, "session copy: %s", hipGetErrorString(e));
  }
  s->graph_enabled = src->graph_enabled;
  s->matrix = src->matrix;  // session options travel with the state
  s->matrix_decode = src->matrix_decode;
  if (src->split_keys != s->split_keys) {
    const int r = cq35_session_set_attention_split(s, src->split_keys);
    if (r) {
      destroy_session(s);
      return r;
    }
  }
  s->mega_on = src->mega_on && s->mega_ok;
  *out = s;
  return CQ35_OK;
}

extern "C" int cq35_session_state_bytes(const cq35_session* s, int which, int64_t* bytes) {
  if (!s || !bytes) return fail(CQ35_EINVAL, "null argument");
  if (which == 0) *bytes = cache_elements(s->model->cfg, s->capacity) * 2;
  else if (which == 1) *bytes = s->model->d.L * s->model->d.REC * 4;
  else if (which == 2 && s->model->cfg.moe) *bytes = s->model->d.L * s->model->d.K * 4;
  else return fail(CQ35_EINVAL, "state buffer %d does not exist", which);
  return CQ35_OK;
}

extern "C" int cq35_session_export_state(const cq35_session* s, int which, void* dst, int64_t bytes) {
  int64_t expect = 0;
  int rc = cq35_session_state_bytes(s, which, &expect);
  if (rc) return rc;
  if (!dst || bytes != expect) return fail(CQ35_EINVAL, "state buffer %d has %lld bytes", which, (long long)expect);
  HIP_TRY(hipSetDevice(s->model->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  const void* src = which == 0 ? (const void*)s->cache : which == 1 ? (const void*)s->shadow : (const void*)s->ids;
  HIP_TRY(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
  return CQ35_OK;
}

extern "C" int cq35_session_import_state(cq35_session* s, int which, const void* src, int64_t bytes) {
  int64_t expect = 0;
  int rc = cq35_session_state_bytes(s, which, &expect);
  if (rc) return rc;
  if (!src || bytes != expect) return fail(CQ35_EINVAL, "state buffer %d has %lld bytes", which, (long long)expect);
  if (which == 2) return fail(CQ35_EINVAL, "state buffer 2 (router top-k) is read-only");
  HIP_TRY(hipSetDevice(s->model->device));
  HIP_TRY(hipStreamSynchronize(s->stream));
  HIP_TRY(hipMemcpy(which == 0 ? (void*)s->cache : (void*)s->shadow, src, bytes, hipMemcpyHostToDevice));
  s->poisoned = false;
  return CQ35_OK;
}

extern "C" int cq35_session_time_kernel(cq35_session* s, int kernel_class) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  if (kernel_class >= KC_COUNT) return fail(CQ35_EINVAL, "unknown kernel class %d", kernel_class);
  HIP_TRY(hipSetDevice(s->model->device));
  if (kernel_class >= 0 && !s->ev[0])
    for (auto& e : s->ev) HIP_TRY(hipEventCreate(&e));
  s->timed_class = kernel_class < 0 ? -1 : kernel_class;
  s->timed_ms = 0.0;
  s->timed_launches = 0;
  s->ev_used = 0;
  return CQ35_OK;
}

extern "C" int cq35_session_kernel_time(cq35_session* s, double* total_ms, int64_t* launches) {
  if (!s || !total_ms || !launches) return fail(CQ35_EINVAL, "null argument");
  *total_ms = s->timed_ms;
  *launches = s->timed_launches;
  return CQ35_OK;
}

extern "C" const char* cq35_kernel_class_name(int kc) {
  return kc >= 0 && kc < KC_COUNT ? kClassNames[kc] : "";
}
extern "C" int cq35_kernel_class_count(void) { return KC_COUNT; }

extern "C" int cq35_session_set_graph(cq35_session* s, int enabled) {
  if (!s) return fail(CQ35_EINVAL, "null argument");
  s->graph_enabled = enabled != 0;
  return CQ35_OK;
}

// ------------------------------------------------------ numeric test hooks

extern "C" float cq35_numeric_exp(float x) { return hexp(x); }
extern "C" float cq35_numeric_sqrt(float x) { return nsqrt(x); }
extern "C" float cq35_numeric_softplus(float x) { return softplus(x); }
extern "C" void cq35_numeric_sincos(float angle, float* sine, float* cosine) {
  sincos_q(angle, sine, cosine);
}

extern "C" int cq35_device_numeric(int op, const float* input, float* output, int64_t count) {
  if (!input || !output || count < 0 || op < 0 || op > 7) return fail(CQ35_EINVAL, "bad argument");
  if (count == 0) return CQ35_OK;
  float *din = nullptr, *dout = nullptr;
  HIP_TRY(hipMalloc(&din, count * 4));
  hipError_t e = hipMalloc(&dout, count * 4);
  if (e == hipSuccess) e = hipMemcpy(din, input, count * 4, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    k_numeric<<<grid_for((count + 255) / 256, 16384), 256>>>(op, din, dout, count);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(output, dout, count * 4, hipMemcpyDeviceToHost);
  hipFree(din);
  if (dout) hipFree(dout);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "device numeric: %s", hipGetErrorString(e));
  return CQ35_OK;
}

extern "C" int cq35_device_gemv(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t cols,
                                int width, uint16_t* out) {
  if (!x || !w || !out || rows <= 0 || cols <= 0 || cols % 2 || rows > (1 << 30) || cols > 32768)
    return fail(CQ35_EINVAL, "bad GEMV shape");
  if (width != 32 && width != 64 && width != 256) return fail(CQ35_EINVAL, "tree width must be 32, 64 or 256");
  // Zero-pad the pairs to a multiple of 4: extra pairs add +-0 to a lane
  // accumulator that is never -0, so every row's value is unchanged.
  const int64_t padded = (cols + 7) / 8 * 8;
  std::vector<uint16_t> xp(padded, 0), wp((size_t)(rows * padded), 0);
  std::copy(x, x + cols, xp.begin());
  for (int64_t r = 0; r < rows; ++r) std::copy(w + r * cols, w + (r + 1) * cols, wp.begin() + r * padded);
  uint16_t *dx = nullptr, *dw = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&dx, padded * 2);
  if (e == hipSuccess) e = hipMalloc(&dw, rows * padded * 2);
  if (e == hipSuccess) e = hipMalloc(&dout, rows * 2);
  if (e == hipSuccess) e = hipMemcpy(dx, xp.data(), padded * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dw, wp.data(), rows * padded * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    Segments seg{};
    seg.w[0] = dw;
    seg.out[0] = dout;
    seg.rows[0] = (int)rows;
    seg.count = 1;
    const int n = (int)padded;
    const size_t lds = (size_t)padded * 2;
    if (width == 32) {
      const unsigned grid = (unsigned)((rows + 31) / 32);
      switch (batch_of((n / 8 + 7) / 8, {8, 16, 32})) {
        case 8: k_project32<false, false, 8><<<grid, kBlock, lds>>>(dx, nullptr, 0.0f, seg, n, nullptr); break;
        case 16: k_project32<false, false, 16><<<grid, kBlock, lds>>>(dx, nullptr, 0.0f, seg, n, nullptr); break;
        default: k_project32<false, false, 32><<<grid, kBlock, lds>>>(dx, nullptr, 0.0f, seg, n, nullptr); break;
      }
    } else if (width == 64) {
      const unsigned grid = (unsigned)((rows + 3) / 4);
      switch (batch_of((n / 8 + 15) / 16, {8, 16, 32})) {
        case 8: k_residual<8><<<grid, 64, lds>>>(dx, dw, (int)rows, n, nullptr, dout); break;
        case 16: k_residual<16><<<grid, 64, lds>>>(dx, dw, (int)rows, n, nullptr, dout); break;
        default: k_residual<32><<<grid, 64, lds>>>(dx, dw, (int)rows, n, nullptr, dout); break;
      }
    } else {
      const unsigned grid = (unsigned)((rows + 4 * kRows256 - 1) / (4 * kRows256));
      k_project256<false><<<grid, kBlock, lds>>>(dx, nullptr, 0.0f, seg, n);
    }
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(out, dout, rows * 2, hipMemcpyDeviceToHost);
  if (dx) hipFree(dx);
  if (dw) hipFree(dw);
  if (dout) hipFree(dout);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "device GEMV: %s", hipGetErrorString(e));
  return CQ35_OK;
}

extern "C" int cq35_device_matrix_gemm(const uint16_t* x, const uint16_t* w, const uint16_t* w2,
                                       const uint16_t* res, int64_t n, int64_t rows, int64_t cols, int mode,
                                       int kernel, uint16_t* out) {
  if (!x || !w || !out || n <= 0 || rows <= 0 || cols <= 0 || cols % 16 || n > (1 << 20) ||
      rows > (1 << 20) || cols > 65536 || mode < kBPlain || mode > kBGate || kernel < 0 || kernel > 1 ||
      (mode == kBGate && !w2) || (mode == kBResidual && !res))
    return fail(CQ35_EINVAL, "bad matrix GEMM shape");
  uint16_t *dx = nullptr, *dw = nullptr, *dw2 = nullptr, *dres = nullptr, *dout = nullptr;
  hipError_t e = hipMalloc(&dx, n * cols * 2);
  if (e == hipSuccess) e = hipMalloc(&dw, rows * cols * 2);
  if (e == hipSuccess && mode == kBGate) e = hipMalloc(&dw2, rows * cols * 2);
  if (e == hipSuccess && mode == kBResidual) e = hipMalloc(&dres, n * rows * 2);
  if (e == hipSuccess) e = hipMalloc(&dout, n * rows * 2);
  if (e == hipSuccess) e = hipMemcpy(dx, x, n * cols * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dw, w, rows * cols * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess && dw2) e = hipMemcpy(dw2, w2, rows * cols * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess && dres) e = hipMemcpy(dres, res, n * rows * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    const int N = (int)n, R = (int)rows, C = (int)cols;
    if (kernel == 0) {
      const dim3 grid((unsigned)((rows + kMRows - 1) / kMRows), (unsigned)((n + kMBlockTokens - 1) / kMBlockTokens));
      if (mode == kBPlain) k_mproject<kBPlain><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
      else if (mode == kBResidual) k_mproject<kBResidual><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
      else k_mproject<kBGate><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
    } else if (cols % (2 * kGBK) == 0) {
      const dim3 grid((unsigned)gemm_grid(R, N));
      const Segments one = segments({{dw, {dout, rows}}});
      if (mode == kBPlain) k_mgemm<kBPlain><<<grid, 64 * kMWaves>>>(dx, N, C, one, dw2, dres);
      else if (mode == kBResidual) k_mgemm<kBResidual><<<grid, 64 * kMWaves>>>(dx, N, C, one, dw2, dres);
      else k_mgemm<kBGate><<<grid, 64 * kMWaves>>>(dx, N, C, one, dw2, dres);
    } else {  // widths the staged tiles do not take run the direct kernel, as in the prefill
      const dim3 grid((unsigned)((rows + kMRows - 1) / kMRows), (unsigned)((n + kMBlockTokens - 1) / kMBlockTokens));
      if (mode == kBPlain) k_mproject<kBPlain><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
      else if (mode == kBResidual) k_mproject<kBResidual><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
      else k_mproject<kBGate><<<grid, 64 * kMWaves>>>(dx, N, C, dw, dw2, R, dres, dout);
    }
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(out, dout, n * rows * 2, hipMemcpyDeviceToHost);
  for (uint16_t* p : {dx, dw, dw2, dres, dout})
    if (p) hipFree(p);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "device matrix GEMM: %s", hipGetErrorString(e));
  return CQ35_OK;
}

extern "C" int cq35_device_matrix_attention(const uint16_t* q, const uint16_t* gate, const uint16_t* k,
                                            const uint16_t* v, int64_t n, int64_t start, int heads,
                                            int kv_heads, int head_dim, uint16_t* out) {
  if (!q || !gate || !k || !v || !out || n <= 0 || start < 0 || n + start > (1 << 20) || heads <= 0 ||
      kv_heads <= 0 || heads > 256 || heads % kv_heads || (head_dim != 64 && head_dim != 128 && head_dim != 256))
    return fail(CQ35_EINVAL, "bad matrix attention shape");
  const int64_t keys = start + n, qs = (int64_t)heads * head_dim, kvs = (int64_t)kv_heads * head_dim;
  uint16_t *dq = nullptr, *dqg = nullptr, *dcache = nullptr, *dout = nullptr;
  uint64_t* dparams = nullptr;
  const uint64_t first_position = (uint64_t)start;
  hipError_t e = hipMalloc(&dq, n * qs * 2);
  if (e == hipSuccess) e = hipMalloc(&dqg, n * 2 * qs * 2);
  if (e == hipSuccess) e = hipMalloc(&dcache, 2 * keys * kvs * 2);
  if (e == hipSuccess) e = hipMalloc(&dout, n * qs * 2);
  if (e == hipSuccess) e = hipMalloc(&dparams, sizeof(uint64_t));
  if (e == hipSuccess) e = hipMemcpy(dq, q, n * qs * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemset(dqg, 0, n * 2 * qs * 2);
  // the projection layout [row][head][q | gate]: gates into the second halves
  if (e == hipSuccess)
    e = hipMemcpy2D(dqg + head_dim, 2 * head_dim * 2, gate, head_dim * 2, head_dim * 2, n * heads,
                    hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dcache, k, keys * kvs * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dcache + keys * kvs, v, keys * kvs * 2, hipMemcpyHostToDevice);
  if (e == hipSuccess) e = hipMemcpy(dparams, &first_position, sizeof(uint64_t), hipMemcpyHostToDevice);
  if (e == hipSuccess) {
    const dim3 grid((unsigned)heads, (unsigned)((n + 31) / 32));
    const float scale = 1.0f / sqrtf((float)head_dim);
    auto run = [&](auto kernel) {
      kernel<<<grid, 64 * kAWaves>>>(dq, dqg, dcache, 0, keys * kvs, dparams, 0, (int)n, (int)kvs, heads,
                                     heads / kv_heads, scale, dout);
    };
    if (head_dim == 256) run(k_mattention<256>);
    else if (head_dim == 128) run(k_mattention<128>);
    else run(k_mattention<64>);
    e = hipGetLastError();
  }
  if (e == hipSuccess) e = hipMemcpy(out, dout, n * qs * 2, hipMemcpyDeviceToHost);
  for (void* p : {(void*)dq, (void*)dqg, (void*)dcache, (void*)dout, (void*)dparams})
    if (p) hipFree(p);
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "device matrix attention: %s", hipGetErrorString(e));
  return CQ35_OK;
}

#include "static_step.h"
