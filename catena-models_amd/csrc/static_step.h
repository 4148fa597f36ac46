// Decode step over caller-owned state that allocates nothing (included at the
// end of runtime.hip; uses its session type and launch sequence).
//
// The per-kernel decode sequence of cq35_step needs scratch beyond its
// inputs and outputs: the step parameters, the argmax key, every activation
// row, the router logits / ids / probabilities and its block ticket, the
// expert activations, the logits row, the RoPE table and the attention
// partials (Q rows of about 3 x capacity floats). Here all of it lives in
// one file-scope device array, `scratch`, of kStaticScratchBytes; each device
// holds its own copy for the life of the process, and its address is taken
// once per device with hipGetSymbolAddress. Calls on one device share the
// array, so each call holds that device's lock from its first launch until
// its stream has drained: calls from several threads (or on several streams)
// of one device run one after another instead of overwriting each other's
// buffers. Nothing but the ticket and the argmax key has to start at zero,
// and both are cleared by a fill kernel at the start of every call. The call
// synchronises its stream and reads the token back before it returns, so it
// cannot be recorded into a captured graph.

namespace cq35 {

constexpr int64_t kStaticScratchBytes = 16ll << 20;

__device__ __align__(256) unsigned char scratch[kStaticScratchBytes];

__global__ void k_clear_words(uint32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

}  // namespace cq35

namespace {

std::mutex g_static_lock;
void* g_static_ptr[64] = {};
// one lock per device, held by a call from its first launch to its final
// stream synchronisation (the calls of one device share its scratch copy)
std::mutex g_static_call[64];

// Device address of `scratch` on the current device (taken once per device).
int static_scratch(int device, unsigned char** out) {
  if (device < 0 || device >= 64) return fail(CQ35_EDEVICE, "device %d out of range", device);
  std::lock_guard<std::mutex> hold(g_static_lock);
  if (!g_static_ptr[device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return fail(CQ35_EDEVICE, "static scratch address: %s", hipGetErrorString(e));
    g_static_ptr[device] = p;
  }
  *out = static_cast<unsigned char*>(g_static_ptr[device]);
  return CQ35_OK;
}

// Carve the per-kernel decode buffers of a session view out of `base`
// (256-byte aligned pieces). Returns the bytes needed; pointers are only
// assigned when base != nullptr.
int64_t static_layout(cq35_session* s, unsigned char* base) {
  const Dims& d = s->model->d;
  const cq35_config& c = s->model->cfg;
  int64_t off = 0;
  auto take = [&](auto** p, int64_t count) {
    using T = std::remove_pointer_t<std::remove_reference_t<decltype(p)>>;
    const int64_t bytes = std::max<int64_t>(count, 1) * (int64_t)sizeof(std::remove_pointer_t<T>);
    if (base) *p = reinterpret_cast<T>(base + off);
    off += (bytes + 255) / 256 * 256;
  };
  // the two words that must start at zero come first (cleared per call)
  take(&s->ticket, 64);
  take(&s->d_best, 2);
  take(&s->d_params, 2);
  take(&s->h, d.H);
  take(&s->attn, d.H);
  take(&s->qkv, d.QKV);
  take(&s->conv, d.QKV);
  take(&s->z, d.VS);
  take(&s->alpha, c.value_heads);
  take(&s->beta, c.value_heads);
  take(&s->gates, c.value_heads);
  take(&s->qn, d.KS);
  take(&s->kn, d.KS);
  take(&s->core, d.VS);
  take(&s->gated, d.VS);
  take(&s->qg, 2 * d.QS);
  take(&s->kraw, d.KVS);
  take(&s->vraw, d.KVS);
  take(&s->qr, d.QS);
  take(&s->ctx, d.QS);
  take(&s->router, d.E + 1);
  take(&s->ids, d.L * std::max<int64_t>(d.K, 1));
  take(&s->probs, std::max<int64_t>(d.K, 1));
  take(&s->active, d.K * d.I + d.SI);
  take(&s->act, d.I);
  take(&s->logits, d.V);
  take(&s->rope, std::max<int64_t>(d.R, 2));
  const int64_t tiles = (s->capacity + 7) / 8;
  s->attn_stride = (int)std::max<int64_t>(tiles * 8 + 2 * tiles + 16, 3 * s->capacity + 16);
  take(&s->attn_scratch, d.Q * (int64_t)s->attn_stride);
  return off;
}

}  // namespace

extern "C" int cq35_step_static(const cq35_model* model, uint16_t* state, int64_t capacity, uint64_t token,
                                int64_t start, void* stream, uint64_t* next_token, uint16_t* logits) {
  if (!model || !state || !next_token) return fail(CQ35_EINVAL, "null argument");
  const cq35_config& c = model->cfg;
  if (capacity <= 0 || capacity > 262144)
    return fail(CQ35_ERANGE, "cache capacity %lld outside 1..262144", (long long)capacity);
  if (start < 0 || start + 1 > capacity)
    return fail(CQ35_ERANGE, "token range %lld..%lld exceeds cache capacity %lld", (long long)start,
                (long long)(start + 1), (long long)capacity);
  if (token >= (uint64_t)c.vocab)
    return fail(CQ35_ERANGE, "token prefix contains an ID outside the %d-token vocabulary", c.vocab);
  HIP_TRY(hipSetDevice(model->device));
  // a view of the caller's state with the session's buffers in `scratch`
  cq35_session view;
  view.model = const_cast<cq35_model*>(model);
  view.capacity = capacity;
  view.cache = state;
  view.stream = static_cast<hipStream_t>(stream);
  view.graph_enabled = false;
  const int64_t need = static_layout(&view, nullptr);
  if (need > kStaticScratchBytes)
    return fail(CQ35_ERANGE,
                "capacity %lld needs %lld bytes of decode scratch; the static maximum is %lld bytes",
                (long long)capacity, (long long)need, (long long)kStaticScratchBytes);
  if (c.moe) {
    // the per-kernel attention and expert kernels' LDS (attributes, not memory)
    const size_t lds = attn_values_lds_bytes(capacity);
    if (lds > 65536 &&
        hipFuncSetAttribute((const void*)k_attn_values, hipFuncAttributeMaxDynamicSharedMemorySize,
                            (int)lds) != hipSuccess)
      return fail(CQ35_EUNSUPPORTED, "capacity %lld needs %zu bytes of LDS for exact-order attention",
                  (long long)capacity, lds);
    if (moe_down_lds_optin(model->d) != hipSuccess)
      return fail(CQ35_EUNSUPPORTED, "expert widths need more LDS than the device grants");
  }
  unsigned char* base = nullptr;
  int rc = static_scratch(model->device, &base);
  if (rc) return rc;
  static_layout(&view, base);
  std::lock_guard<std::mutex> serial(g_static_call[model->device]);
  const uint64_t params[2] = {(uint64_t)start, token};
  unsigned long long key = 0;
  hipError_t e = hipSuccess;
  k_clear_words<<<1, 64, 0, view.stream>>>(reinterpret_cast<uint32_t*>(view.ticket), 64);
  k_clear_words<<<1, 64, 0, view.stream>>>(reinterpret_cast<uint32_t*>(view.d_best), 4);
  e = hipGetLastError();
  if (e == hipSuccess)
    e = hipMemcpyAsync(view.d_params, params, sizeof(params), hipMemcpyHostToDevice, view.stream);
  if (e == hipSuccess) {
    enqueue_token(&view, 0, true, false);
    e = hipGetLastError();
  }
  if (e == hipSuccess)
    e = hipMemcpyAsync(&key, view.d_best, sizeof(key), hipMemcpyDeviceToHost, view.stream);
  if (e == hipSuccess && logits)
    e = hipMemcpyAsync(logits, view.logits, (size_t)c.vocab * 2, hipMemcpyDeviceToHost, view.stream);
  if (e == hipSuccess) e = hipStreamSynchronize(view.stream);
  view.stream = nullptr;  // the caller's: not destroyed with the view
  if (e != hipSuccess) return fail(CQ35_EDEVICE, "static step: %s", hipGetErrorString(e));
  const uint64_t t = decode_key(key);
  if (t >= (uint64_t)c.vocab)
    return fail(CQ35_EDEVICE, "qwen3 returned next-token ID %llu outside the vocabulary", (unsigned long long)t);
  *next_token = t;
  return CQ35_OK;
}
