// gdn_exec.cpp -- the executor: ModelExecutor (src/scheduler/executor.rs:21-49)
// over pool slots, written against the public C ABI of the layers it drives
// (gdn_layer_*, gdn_qlinear_*, gdn_slot_*), the way a host-language executor
// would bind it.
//
// Per sequence the reference keeps Qwen35State { caches: Vec<(conv, state)> }
// (mlx_executor.rs:19-21) and copies every active sequence's caches into a
// batch and back on every step (stack_caches / unstack_caches, :92-130).
// Here a sequence is one slot id, the same in every layer: a decode step
// stages B (slot, token) pairs, and the layers read and write the slots in
// place. Device work of a step, in stream order:
//   H2D of the (slot, token) block -> embedding rows -> per layer: residual
//   add + rms-norm, gdn_layer_decode -> final add + norm -> lm_head -> argmax
//   -> D2H of the B picked tokens, then an event that collect waits for.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "gdn.h"
#include "gdn_common.h"

namespace {

gdn_status efail(gdn_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return gdn::set_error(code, buf);
}

gdn_status hfail(hipError_t e, const char* what) {
  return efail(GDN_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

#define GDN_TRY(x)                      \
  do {                                  \
    gdn_status st_ = (x);               \
    if (st_ != GDN_OK) return st_;      \
  } while (0)
#define HIP_TRY(x, what)                  \
  do {                                    \
    hipError_t e_ = (x);                  \
    if (e_ != hipSuccess) return hfail(e_, what); \
  } while (0)

}  // namespace

struct gdn_exec {
  gdn_pool* pool = nullptr;
  std::vector<gdn_layer*> layers;
  std::vector<const uint16_t*> norm_w;
  const uint16_t* final_norm_w = nullptr;
  float eps = 0.f;
  const uint16_t* embed = nullptr;
  const gdn_qlinear* head = nullptr;
  int hidden = 0, vocab = 0, max_batch = 0, max_prompt = 0, rows = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t done = nullptr;
  // device buffers
  int32_t* d_dec = nullptr;   // [2 * max_batch]: slots, then tokens
  int32_t* d_pre = nullptr;   // [3 + max_prompt]: slot, cu[0..1], prompt
  int32_t* d_next = nullptr;  // [max_batch] picked tokens
  uint16_t* h = nullptr;      // residual stream [rows, hidden]
  uint16_t* hn = nullptr;     // normed rows fed to a layer
  uint16_t* mix = nullptr;    // layer output rows
  uint16_t* logits = nullptr; // [max_batch, vocab]
  float* d_pv = nullptr;      // greedy-pick partials [max_batch, argmax_chunks(vocab)]
  int* d_pi = nullptr;
  // pinned host staging (one region per direction and kind, so a prefill
  // staged while a batch is in flight does not overwrite it)
  int32_t* p_dec = nullptr;
  int32_t* p_pre = nullptr;
  int32_t* p_next = nullptr;   // a batch's picked tokens
  int32_t* p_first = nullptr;  // a prefill's first token
  std::unordered_map<uint64_t, int32_t> slot_of;
  bool inflight = false;
  int32_t inflight_B = 0;
  int32_t logits_rows = 0;
};

namespace {

void exec_release(gdn_exec* x) {
  if (!x) return;
  if (x->stream) (void)hipStreamSynchronize(x->stream);
  for (void* p : {(void*)x->d_dec, (void*)x->d_pre, (void*)x->d_next, (void*)x->h, (void*)x->hn,
                  (void*)x->mix, (void*)x->logits, (void*)x->d_pv, (void*)x->d_pi})
    if (p) (void)hipFree(p);
  for (void* p : {(void*)x->p_dec, (void*)x->p_pre, (void*)x->p_next, (void*)x->p_first})
    if (p) (void)hipHostFree(p);
  if (x->done) (void)hipEventDestroy(x->done);
  for (auto& kv : x->slot_of) (void)gdn_slot_free(x->pool, kv.second);
  delete x;
}

// Makes the executor's device current for the duration of a call.
struct DevScope {
  int prev = -1;
  explicit DevScope(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
  }
  ~DevScope() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

// The model body over n rows of h that hold the embedded tokens: every GDN
// layer with its residual seam, then the final norm into hn.
gdn_status run_layers(gdn_exec* x, int n, bool prefill) {
  const int32_t* slots = prefill ? x->d_pre : x->d_dec;
  for (size_t l = 0; l < x->layers.size(); ++l) {
    HIP_TRY(gdn::launch_add_norm(x->h, l == 0 ? nullptr : x->mix, n, x->hidden, x->norm_w[l],
                                 x->eps, x->hn, x->stream),
            "residual add + norm");
    if (prefill)
      GDN_TRY(gdn_layer_prefill(x->layers[l], slots, x->d_pre + 1, 1, n, x->hn, x->hidden, x->mix,
                                x->hidden, x->stream));
    else
      GDN_TRY(gdn_layer_decode(x->layers[l], slots, n, x->hn, x->hidden, x->mix, x->hidden,
                               x->stream));
  }
  return GDN_OK;
}

// lm_head + argmax of n rows starting at row r0 of h (after the last
// layer's residual add), picked tokens into d_next and the pinned `dst`.
gdn_status pick(gdn_exec* x, int r0, int n, int32_t* dst) {
  uint16_t* hr = x->h + (size_t)r0 * x->hidden;
  const uint16_t* mr = x->layers.empty() ? nullptr : x->mix + (size_t)r0 * x->hidden;
  uint16_t* nr = x->hn + (size_t)r0 * x->hidden;
  HIP_TRY(gdn::launch_add_norm(hr, mr, n, x->hidden, x->final_norm_w, x->eps, nr, x->stream),
          "final norm");
  GDN_TRY(gdn_qlinear_forward(x->head, nr, x->hidden, n, x->logits, x->vocab, x->stream));
  HIP_TRY(gdn::launch_argmax(x->logits, x->vocab, n, x->vocab, x->d_pv, x->d_pi, x->d_next,
                             x->stream),
          "argmax");
  HIP_TRY(hipMemcpyAsync(dst, x->d_next, sizeof(int32_t) * n, hipMemcpyDeviceToHost, x->stream),
          "token copy");
  x->logits_rows = n;
  return GDN_OK;
}

}  // namespace

extern "C" {

gdn_status gdn_exec_create(const gdn_exec_desc* desc, void* stream, gdn_exec** out) {
  if (!desc || !out) return efail(GDN_ERR_INVALID, "gdn_exec_create: desc/out is NULL");
  *out = nullptr;
  const gdn_exec_desc& d = *desc;
  if (!d.pool || !d.embed || !d.head || !d.final_norm_w || d.num_layers < 0 ||
      (d.num_layers > 0 && (!d.layers || !d.input_norm_w)))
    return efail(GDN_ERR_INVALID, "gdn_exec_create: NULL pool / embed / head / norm / layers");
  for (int l = 0; l < d.num_layers; ++l)
    if (!d.layers[l] || !d.input_norm_w[l])
      return efail(GDN_ERR_INVALID, "gdn_exec_create: layer %d or its norm weight is NULL", l);
  if (d.max_batch < 1 || d.max_prompt < 1)
    return efail(GDN_ERR_INVALID, "gdn_exec_create: max_batch and max_prompt must be >= 1");
  if (!(d.rms_eps >= 0.0f)) return efail(GDN_ERR_INVALID, "gdn_exec_create: rms_eps < 0");
  if (reinterpret_cast<uintptr_t>(d.embed) % 16 != 0)
    return efail(GDN_ERR_INVALID, "gdn_exec_create: embed must be 16-byte aligned");
  int32_t hidden = 0, vocab = 0;
  GDN_TRY(gdn_qlinear_dims(d.head, &hidden, &vocab));
  if (hidden > 4096) return efail(GDN_ERR_UNSUPPORTED, "gdn_exec_create: hidden %d > 4096", hidden);
  DevScope dev(d.device);
  gdn_exec* x = new gdn_exec;
  x->pool = d.pool;
  x->layers.assign(d.layers, d.layers + d.num_layers);
  x->norm_w.assign(d.input_norm_w, d.input_norm_w + d.num_layers);
  x->final_norm_w = d.final_norm_w;
  x->eps = d.rms_eps;
  x->embed = d.embed;
  x->head = d.head;
  x->hidden = hidden;
  x->vocab = vocab;
  x->max_batch = d.max_batch;
  x->max_prompt = d.max_prompt;
  x->rows = d.max_batch > d.max_prompt ? d.max_batch : d.max_prompt;
  x->device = d.device;
  x->stream = static_cast<hipStream_t>(stream);
  const size_t act = (size_t)x->rows * hidden * sizeof(uint16_t);
  bool ok = hipMalloc(&x->d_dec, sizeof(int32_t) * 2 * d.max_batch) == hipSuccess &&
            hipMalloc(&x->d_pre, sizeof(int32_t) * (3 + (size_t)d.max_prompt)) == hipSuccess &&
            hipMalloc(&x->d_next, sizeof(int32_t) * d.max_batch) == hipSuccess &&
            hipMalloc(&x->h, act) == hipSuccess && hipMalloc(&x->hn, act) == hipSuccess &&
            hipMalloc(&x->mix, act) == hipSuccess &&
            hipMalloc(&x->logits, (size_t)d.max_batch * vocab * sizeof(uint16_t)) == hipSuccess &&
            hipMalloc(&x->d_pv, sizeof(float) * d.max_batch * gdn::argmax_chunks(vocab)) == hipSuccess &&
            hipMalloc(&x->d_pi, sizeof(int) * d.max_batch * gdn::argmax_chunks(vocab)) == hipSuccess &&
            hipHostMalloc(&x->p_dec, sizeof(int32_t) * 2 * d.max_batch, 0) == hipSuccess &&
            hipHostMalloc(&x->p_pre, sizeof(int32_t) * (3 + (size_t)d.max_prompt), 0) == hipSuccess &&
            hipHostMalloc(&x->p_next, sizeof(int32_t) * d.max_batch, 0) == hipSuccess &&
            hipHostMalloc(&x->p_first, sizeof(int32_t), 0) == hipSuccess &&
            hipEventCreateWithFlags(&x->done, hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    (void)hipGetLastError();
    exec_release(x);
    return efail(GDN_ERR_OOM, "gdn_exec_create: buffers for %d rows x %d hidden", x->rows, hidden);
  }
  // size the layers' activation buffer once: later calls allocate nothing
  gdn_status st = gdn_pool_reserve(d.pool, x->rows, stream);
  if (st != GDN_OK) {
    exec_release(x);
    return st;
  }
  *out = x;
  return GDN_OK;
}

gdn_status gdn_exec_destroy(gdn_exec* x) {
  exec_release(x);
  return GDN_OK;
}

gdn_status gdn_exec_prefill(gdn_exec* x, uint64_t seq_id, const int32_t* prompt, int32_t len,
                            uint32_t* first_token) {
  if (!x || !prompt || !first_token) return efail(GDN_ERR_INVALID, "gdn_exec_prefill: NULL argument");
  if (len < 1 || len > x->max_prompt)
    return efail(GDN_ERR_INVALID, "gdn_exec_prefill: prompt length %d outside [1, %d]", len,
                 x->max_prompt);
  for (int i = 0; i < len; ++i)
    if (prompt[i] < 0 || prompt[i] >= x->vocab)
      return efail(GDN_ERR_INVALID, "gdn_exec_prefill: token %d at %d outside [0, %d)", prompt[i],
                   i, x->vocab);
  DevScope dev(x->device);
  // admit: a fresh sequence gets a free slot; a known one starts over
  int32_t slot;
  auto it = x->slot_of.find(seq_id);
  if (it != x->slot_of.end()) {
    slot = it->second;
  } else {
    if (gdn_slot_alloc(x->pool, &slot) != GDN_OK)
      return efail(GDN_ERR_SLOTS, "gdn_exec_prefill: no free slot for sequence %llu",
                   (unsigned long long)seq_id);
    x->slot_of.emplace(seq_id, slot);
  }
  // the pinned prefill block may still feed an earlier prefill's copy only if
  // that call failed half-way; prefill syncs at its end, so it is free here
  x->p_pre[0] = slot;
  x->p_pre[1] = 0;
  x->p_pre[2] = len;
  for (int i = 0; i < len; ++i) x->p_pre[3 + i] = prompt[i];
  HIP_TRY(hipMemcpyAsync(x->d_pre, x->p_pre, sizeof(int32_t) * (3 + (size_t)len),
                         hipMemcpyHostToDevice, x->stream),
          "prompt copy");
  GDN_TRY(gdn_slots_zero(x->pool, GDN_ALL_LAYERS, x->d_pre, 1, x->stream));
  HIP_TRY(gdn::launch_embed(x->embed, x->d_pre + 3, len, x->vocab, x->hidden, x->h, x->stream),
          "embedding");
  GDN_TRY(run_layers(x, len, true));
  GDN_TRY(pick(x, len - 1, 1, x->p_first));
  HIP_TRY(hipStreamSynchronize(x->stream), "gdn_exec_prefill sync");
  *first_token = (uint32_t)x->p_first[0];
  return GDN_OK;
}

gdn_status gdn_exec_submit_batch(gdn_exec* x, const uint64_t* seq_ids, const uint32_t* tokens,
                                 int32_t B) {
  if (!x) return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: NULL executor");
  if (x->inflight)
    return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: a submitted batch is not collected yet");
  if (B < 1 || B > x->max_batch)
    return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: B = %d outside [1, %d]", B,
                 x->max_batch);
  if (!seq_ids || !tokens) return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: NULL argument");
  std::unordered_set<uint64_t> seen;
  for (int b = 0; b < B; ++b) {
    auto it = x->slot_of.find(seq_ids[b]);
    if (it == x->slot_of.end())
      return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: sequence %llu was not prefilled",
                   (unsigned long long)seq_ids[b]);
    if (!seen.insert(seq_ids[b]).second)
      return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: sequence %llu appears twice",
                   (unsigned long long)seq_ids[b]);
    if (tokens[b] >= (uint32_t)x->vocab)
      return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: token %u outside [0, %d)", tokens[b],
                   x->vocab);
    x->p_dec[b] = it->second;
    x->p_dec[x->max_batch + b] = (int32_t)tokens[b];
  }
  DevScope dev(x->device);
  HIP_TRY(hipMemcpyAsync(x->d_dec, x->p_dec, sizeof(int32_t) * 2 * x->max_batch,
                         hipMemcpyHostToDevice, x->stream),
          "batch copy");
  HIP_TRY(gdn::launch_embed(x->embed, x->d_dec + x->max_batch, B, x->vocab, x->hidden, x->h,
                            x->stream),
          "embedding");
  GDN_TRY(run_layers(x, B, false));
  GDN_TRY(pick(x, 0, B, x->p_next));
  HIP_TRY(hipEventRecord(x->done, x->stream), "gdn_exec_submit_batch event");
  x->inflight = true;
  x->inflight_B = B;
  return GDN_OK;
}

gdn_status gdn_exec_collect_batch(gdn_exec* x, uint32_t* next_tokens, int32_t B) {
  if (!x || !next_tokens) return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: NULL argument");
  if (!x->inflight) return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: nothing submitted");
  if (B != x->inflight_B)
    return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: B = %d, submitted %d", B,
                 x->inflight_B);
  x->inflight = false;
  HIP_TRY(hipEventSynchronize(x->done), "gdn_exec_collect_batch");
  for (int b = 0; b < B; ++b) next_tokens[b] = (uint32_t)x->p_next[b];
  return GDN_OK;
}

gdn_status gdn_exec_decode_batch(gdn_exec* x, const uint64_t* seq_ids, const uint32_t* tokens,
                                 int32_t B, uint32_t* next_tokens) {
  GDN_TRY(gdn_exec_submit_batch(x, seq_ids, tokens, B));
  return gdn_exec_collect_batch(x, next_tokens, B);
}

gdn_status gdn_exec_release(gdn_exec* x, uint64_t seq_id) {
  if (!x) return efail(GDN_ERR_INVALID, "gdn_exec_release: NULL executor");
  auto it = x->slot_of.find(seq_id);
  if (it == x->slot_of.end())
    return efail(GDN_ERR_INVALID, "gdn_exec_release: unknown sequence %llu",
                 (unsigned long long)seq_id);
  // Work already queued on the slot runs before any later prefill re-zeroes
  // it (one stream), so the slot can be handed out again at once.
  GDN_TRY(gdn_slot_free(x->pool, it->second));
  x->slot_of.erase(it);
  return GDN_OK;
}

int32_t gdn_exec_max_batch_size(const gdn_exec* x) { return x ? x->max_batch : 0; }

int32_t gdn_exec_supports_pipeline(const gdn_exec* x) { return x ? 1 : 0; }

gdn_status gdn_exec_seq_slot(const gdn_exec* x, uint64_t seq_id, int32_t* slot) {
  if (!x || !slot) return efail(GDN_ERR_INVALID, "gdn_exec_seq_slot: NULL argument");
  auto it = x->slot_of.find(seq_id);
  if (it == x->slot_of.end())
    return efail(GDN_ERR_INVALID, "gdn_exec_seq_slot: unknown sequence %llu",
                 (unsigned long long)seq_id);
  *slot = it->second;
  return GDN_OK;
}

gdn_status gdn_exec_logits(const gdn_exec* x, const uint16_t** logits, int32_t* rows,
                           int32_t* vocab) {
  if (!x || !logits || !rows || !vocab) return efail(GDN_ERR_INVALID, "gdn_exec_logits: NULL argument");
  *logits = x->logits;
  *rows = x->logits_rows;
  *vocab = x->vocab;
  return GDN_OK;
}

}  // extern "C"
