// gdn_exec.cpp -- the executor: ModelExecutor (src/scheduler/executor.rs:21-49)
// over pool slots, written against the public C ABI of the layers it drives
// (gdn_layer_*, gdn_qlinear_*, gdn_slot_*, gdn_kv_*, gdn_attn_forward), the
// way a host-language executor would bind it.
//
// Per sequence the reference keeps Qwen35State { caches: Vec<(conv, state)> }
// (mlx_executor.rs:19-21) and copies every active sequence's caches into a
// batch and back on every step (stack_caches / unstack_caches, :92-130).
// Here a sequence is one slot id, the same in every layer: a decode step
// stages B (slot, token) pairs, and the layers read and write the slots in
// place; the attention layers' KV cache (when the stack has attention layers)
// is keyed by the same slot ids and planned once per step (gdn_kv_step).
// Device work of a step, in stream order:
//   H2D of the (slot, token) block -> per decoder layer: residual add +
//   rms-norm (the first one reading the embedding rows), then
//   gdn_layer_decode (GDN) or q|k|v projection, gdn_attn_forward and o_proj
//   (attention) -> final add + norm -> lm_head -> argmax into the token half
//   of the device (slot, token) block and into a device-mapped pinned host
//   slot, which collect polls (the host clears it to -1 before the step).
// Since the picks land where the next step's embedding reads its tokens, a
// chained step (gdn_exec_submit_next) is the same device work without the H2D
// copy, queued while the step before it still runs: the double-buffered decode
// of src/bin/qwen_mlx_infer.rs:136-187, which builds step N+1 on step N's
// unevaluated token array.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <string>
#include <chrono>
#include <thread>
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
  struct Attn {
    const gdn_qlinear* qkv;
    const gdn_qlinear* o;
    const uint16_t* q_norm_w;
    const uint16_t* k_norm_w;
  };
  gdn_pool* pool = nullptr;
  std::vector<gdn_layer*> layers;
  std::vector<Attn> attn;
  // decoder stack: entry >= 0 is GDN layer entry, < 0 attention layer -entry - 1
  std::vector<int> stack;
  std::vector<const uint16_t*> norm_w;  // per stack position
  gdn_kv* kv = nullptr;
  float rope_theta = 0.f;
  int rotary_dim = 0, Hq = 0, Hkv = 0, nqkv = 0;
  const uint16_t* final_norm_w = nullptr;
  float eps = 0.f;
  const uint16_t* embed = nullptr;
  const gdn_qlinear* head = nullptr;
  int hidden = 0, vocab = 0, max_batch = 0, max_prompt = 0, rows = 0;
  int device = 0;
  hipStream_t stream = nullptr;
  hipEvent_t pre_copied = nullptr;   // the prefill block has left p_pre
  // device buffers
  int32_t* d_dec = nullptr;   // [2 * max_batch]: slots, then tokens (a step's picks replace them)
  int32_t* d_pre = nullptr;   // prefill block, pre_words(): slots, cu, last rows, tokens
  int32_t* d_next = nullptr;  // [max_batch] a prefill's picked tokens
  uint16_t* h = nullptr;      // residual stream [rows, hidden]
  uint16_t* hn = nullptr;     // normed rows fed to a layer
  uint16_t* mix = nullptr;    // layer output rows
  uint16_t* xsplit = nullptr; // group sums of <= 64 normed rows, split in three [3][64][hidden/64]
  gdn::QPartial pend{};       // the last mixer's output as pending K-slice partials (in place
                              // of mix rows when nslice > 0), added by the next residual seam
  uint16_t* logits = nullptr; // [max_batch, vocab]
  uint16_t* qkv = nullptr;    // attention q|gate, k, v rows [rows, nqkv]
  uint16_t* att = nullptr;    // gated attention rows [rows, Hq * 256]
  float* d_pv = nullptr;      // greedy-pick partials [max_batch, argmax_chunks(vocab)]
  int* d_pi = nullptr;
  // pinned host staging (one region per direction and kind, so a prefill
  // staged while a batch is in flight does not overwrite it)
  int32_t* p_dec = nullptr;
  int32_t* p_pre = nullptr;
  int32_t* p_next = nullptr;   // [2 * max_batch] picked tokens of the uncollected steps
  int32_t* p_next_dev = nullptr;  // p_next as the device addresses it (written by argmax)
  int32_t* p_first = nullptr;  // a prefill's first tokens [max_batch]
  std::vector<int32_t> ones;   // ntok = 1 per decode sequence
  std::unordered_map<uint64_t, int32_t> slot_of;
  // uncollected decode steps, oldest first: pend_n of them from ring entry pend_head
  int pend_n = 0, pend_head = 0;
  int32_t pend_B[2] = {0, 0};
  int32_t chain_B = 0;  // rows of the last submitted step a chained step may follow (0: none)
  int32_t logits_rows = 0;
  // Decode steps replay HIP graphs, one per batch size: the step's launches
  // between attention calls captured once as segments (an attention call's
  // launch shape follows the step's KV plan, so it runs eagerly between them).
  bool use_graphs = true;
  bool use_split_sums = true;  // in_proj and lm_head take their rows' group sums from the norm
  hipStream_t cap = nullptr;  // private stream the segments are captured on
  struct StepGraphs {
    std::vector<hipGraphExec_t> seg[2];  // per pinned pick slot the step writes
    bool failed = false;  // capture refused (e.g. a debug check syncing): run eagerly
  };
  std::unordered_map<int32_t, StepGraphs> graphs;
  uint64_t graphs_act_gen = 0;  // the pool's activation buffer the graphs were captured on
};

namespace {

void exec_release(gdn_exec* x) {
  if (!x) return;
  if (x->stream) (void)hipStreamSynchronize(x->stream);
  else (void)hipDeviceSynchronize();
  for (auto& kv : x->graphs)
    for (auto& v : kv.second.seg)
      for (hipGraphExec_t g : v) (void)hipGraphExecDestroy(g);
  if (x->cap) (void)hipStreamDestroy(x->cap);
  for (void* p : {(void*)x->d_dec, (void*)x->d_pre, (void*)x->d_next, (void*)x->h, (void*)x->hn,
                  (void*)x->mix, (void*)x->xsplit, (void*)x->logits, (void*)x->d_pv, (void*)x->d_pi, (void*)x->qkv,
                  (void*)x->att})
    if (p) (void)hipFree(p);
  for (void* p : {(void*)x->p_dec, (void*)x->p_pre, (void*)x->p_next, (void*)x->p_first})
    if (p) (void)hipHostFree(p);
  if (x->pre_copied) (void)hipEventDestroy(x->pre_copied);
  for (auto& sv : x->slot_of) {
    (void)gdn_slot_free(x->pool, sv.second);
    if (x->kv) (void)gdn_kv_release(x->kv, sv.second);
  }
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

// Words of the pinned / device prefill block: nseq slots, nseq + 1 cu_seqlens,
// nseq last-row indices (at most max_batch sequences each), then the packed
// prompt tokens (at most max_prompt).
size_t pre_words(int max_batch, int max_prompt) {
  return 3 * (size_t)max_batch + 1 + (size_t)max_prompt;
}

// The first seam of the stack: h = the embedding rows of toks, hn = its
// rms-norm; later seams add the previous mixer's output first. xsp (or null):
// also hn's split group sums, for the next in_proj.
gdn_status seam(gdn_exec* x, size_t p, int n, const int32_t* toks, uint16_t* xsp = nullptr) {
  if (p == 0)
    HIP_TRY(gdn::launch_embed_norm(x->embed, toks, n, x->vocab, x->hidden, x->norm_w[0], x->eps,
                                   x->h, x->hn, x->stream, xsp),
            "embedding + norm");
  else
    HIP_TRY(gdn::launch_add_norm(x->h, x->mix, &x->pend, n, x->hidden, x->norm_w[p], x->eps,
                                 x->hn, x->stream, xsp),
            "residual add + norm");
  x->pend = gdn::QPartial{};
  return GDN_OK;
}

// The model body over n rows of the tokens toks: every decoder layer with its
// residual seam (an empty stack only embeds). Prefill rows are nseq packed
// sequences. The KV step for these rows is planned before this runs.
gdn_status run_layers(gdn_exec* x, int n, bool prefill, const int32_t* toks, int nseq = 0) {
  const int32_t* slots = prefill ? x->d_pre : x->d_dec;
  const int qw = 2 * x->Hq * 256, kw = x->Hkv * 256;  // q|gate and k widths of a qkv row
  if (x->stack.empty())
    HIP_TRY(gdn::launch_embed(x->embed, toks, n, x->vocab, x->hidden, x->h, x->stream),
            "embedding");
  for (size_t p = 0; p < x->stack.size(); ++p) {
    GDN_TRY(seam(x, p, n, toks));
    const int e = x->stack[p];
    if (e < 0) {
      const int ai = -e - 1;
      const gdn_exec::Attn& a = x->attn[ai];
      GDN_TRY(gdn_qlinear_forward(a.qkv, x->hn, x->hidden, n, x->qkv, x->nqkv, x->stream));
      GDN_TRY(gdn_attn_forward(x->kv, ai, x->qkv, x->nqkv, x->qkv + qw, x->nqkv, x->qkv + qw + kw,
                               x->nqkv, a.q_norm_w, a.k_norm_w, x->eps, x->rope_theta,
                               x->rotary_dim, x->att, x->Hq * 256, x->stream));
      GDN_TRY(gdn::qlinear_forward(a.o, x->att, x->Hq * 256, n, x->mix, x->hidden, x->stream,
                                   &x->pend));
    } else if (prefill) {
      GDN_TRY(gdn_layer_prefill(x->layers[e], slots, x->d_pre + nseq, nseq, n, x->hn, x->hidden,
                                x->mix, x->hidden, x->stream));
    } else {
      GDN_TRY(gdn::layer_decode(x->layers[e], slots, n, x->hn, x->hidden, x->mix, x->hidden,
                                x->stream, &x->pend));
    }
  }
  return GDN_OK;
}

// One attention layer's gdn_attn_forward on rows already projected into qkv.
gdn_status attn_call(gdn_exec* x, int ai) {
  const gdn_exec::Attn& a = x->attn[ai];
  const int qw = 2 * x->Hq * 256, kw = x->Hkv * 256;
  return gdn_attn_forward(x->kv, ai, x->qkv, x->nqkv, x->qkv + qw, x->nqkv, x->qkv + qw + kw,
                          x->nqkv, a.q_norm_w, a.k_norm_w, x->eps, x->rope_theta, x->rotary_dim,
                          x->att, x->Hq * 256, x->stream);
}

// Segment k of a decode step over B rows (segments end at each attention
// call): segment 0 starts with the embedding, every segment but the last ends
// with an attention layer's q|k|v projection, the next one starts with its
// output projection, and the last ends with lm_head and the greedy pick into
// the token half of d_dec and into pinned pick slot ps. The segments and the
// attention calls between them, in order, are the step.
gdn_status decode_seg(gdn_exec* x, int B, int k, int ps) {
  int32_t* const toks = x->d_dec + x->max_batch;
  int seg = 0;
  if (k == 0 && x->stack.empty())
    HIP_TRY(gdn::launch_embed(x->embed, toks, B, x->vocab, x->hidden, x->h, x->stream),
            "embedding");
  for (size_t p = 0; p < x->stack.size(); ++p) {
    const int e = x->stack[p];
    if (seg == k) {
      // a GDN layer's in_proj takes the group sums of its rows from the seam
      uint16_t* const xsp =
          x->use_split_sums && e >= 0 && B <= 64 && x->hidden % 64 == 0 ? x->xsplit : nullptr;
      GDN_TRY(seam(x, p, B, toks, xsp));
      if (e >= 0) {
        GDN_TRY(gdn::layer_decode(x->layers[e], x->d_dec, B, x->hn, x->hidden, x->mix, x->hidden,
                                  x->stream, &x->pend, xsp));
      } else {
        GDN_TRY(gdn_qlinear_forward(x->attn[-e - 1].qkv, x->hn, x->hidden, B, x->qkv, x->nqkv,
                                    x->stream));
      }
    }
    if (e < 0) {
      ++seg;
      if (seg == k)
        GDN_TRY(gdn::qlinear_forward(x->attn[-e - 1].o, x->att, x->Hq * 256, B, x->mix, x->hidden,
                                     x->stream, &x->pend));
    }
  }
  if (seg != k) return GDN_OK;
  gdn::QPartial pp = x->pend;
  // lm_head, too, takes its rows' group sums from the norm
  uint16_t* const hxs = x->use_split_sums && B <= 64 && x->hidden % 64 == 0 ? x->xsplit : nullptr;
  HIP_TRY(gdn::launch_add_norm(x->h, x->stack.empty() ? nullptr : x->mix,
                               x->stack.empty() ? nullptr : &pp, B, x->hidden, x->final_norm_w,
                               x->eps, x->hn, x->stream, hxs),
          "final norm");
  x->pend = gdn::QPartial{};
  GDN_TRY(gdn::qlinear_forward(x->head, x->hn, x->hidden, B, x->logits, x->vocab, x->stream,
                               nullptr, hxs));
  // the picks overwrite the step's input tokens (the embedding has read them)
  HIP_TRY(gdn::launch_argmax(x->logits, x->vocab, B, x->vocab, x->d_pv, x->d_pi, toks,
                             x->p_next_dev + (size_t)ps * x->max_batch, x->stream),
          "argmax");
  return GDN_OK;
}

// Captures the B-row decode step's segments into graphs, one set per pinned
// pick slot (once per B). A capture that fails leaves the batch size on the
// eager path.
// Drops every captured step graph (they hold the pool's activation buffer,
// which a layer call with more rows or gdn_pool_reserve may have reallocated).
void drop_graphs(gdn_exec* x) {
  if (x->graphs.empty()) return;
  (void)hipStreamSynchronize(x->stream);  // no replay still in flight
  for (auto& kv : x->graphs)
    for (auto& v : kv.second.seg)
      for (hipGraphExec_t g : v) (void)hipGraphExecDestroy(g);
  x->graphs.clear();
}

gdn_exec::StepGraphs& step_graphs(gdn_exec* x, int B) {
  const uint64_t gen = gdn::pool_act_generation(x->pool);
  if (gen != x->graphs_act_gen) {
    drop_graphs(x);
    x->graphs_act_gen = gen;
  }
  gdn_exec::StepGraphs& sg = x->graphs[B];
  if (!sg.seg[0].empty() || sg.failed) return sg;
  const int nseg = (int)x->attn.size() + 1;
  if (!x->cap && hipStreamCreateWithFlags(&x->cap, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    sg.failed = true;
    return sg;
  }
  hipStream_t saved = x->stream;
  x->stream = x->cap;
  const gdn::QPartial pend0 = x->pend;
  for (int ps = 0; ps < 2; ++ps)
    for (int k = 0; k < nseg && !sg.failed; ++k) {
      hipGraph_t g = nullptr;
      hipGraphExec_t ge = nullptr;
      if (hipStreamBeginCapture(x->cap, hipStreamCaptureModeThreadLocal) != hipSuccess) {
        sg.failed = true;
        break;
      }
      const gdn_status st = decode_seg(x, B, k, ps);
      const hipError_t e = hipStreamEndCapture(x->cap, &g);
      if (st != GDN_OK || e != hipSuccess || !g ||
          hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess)
        sg.failed = true;
      else
        sg.seg[ps].push_back(ge);
      if (g) (void)hipGraphDestroy(g);
    }
  x->stream = saved;
  x->pend = pend0;
  if (sg.failed) {
    (void)hipGetLastError();
    for (auto& v : sg.seg) {
      for (hipGraphExec_t ge : v) (void)hipGraphExecDestroy(ge);
      v.clear();
    }
  }
  return sg;
}

// Queues the device work of a decode step over the B rows of the device
// (slot, token) block, its picks going to the next free pinned slot, cleared
// to -1 first (no device work writes it: its last step was collected). The
// attention layers' KV step is planned already.
gdn_status queue_step(gdn_exec* x, int32_t B) {
  const int nseg = (int)x->attn.size() + 1;
  const int e = (x->pend_head + x->pend_n) & 1;
  volatile int32_t* slot = x->p_next + (size_t)e * x->max_batch;
  for (int b = 0; b < B; ++b) slot[b] = -1;
  gdn_exec::StepGraphs* sg = x->use_graphs ? &step_graphs(x, B) : nullptr;
  const bool replay = sg && !sg->seg[e].empty();
  for (int k = 0; k < nseg; ++k) {
    if (replay)
      HIP_TRY(hipGraphLaunch(sg->seg[e][k], x->stream), "decode step graph");
    else
      GDN_TRY(decode_seg(x, B, k, e));
    if (k + 1 < nseg) GDN_TRY(attn_call(x, k));
  }
  x->logits_rows = B;
  x->pend_B[e] = B;
  ++x->pend_n;
  x->chain_B = B;
  return GDN_OK;
}

}  // namespace

extern "C" {

gdn_status gdn_exec_create(const gdn_exec_desc* desc, void* stream, gdn_exec** out) {
  if (!desc || !out) return efail(GDN_ERR_INVALID, "gdn_exec_create: desc/out is NULL");
  *out = nullptr;
  const gdn_exec_desc& d = *desc;
  if (!d.pool || !d.embed || !d.head || !d.final_norm_w || d.num_layers < 0 ||
      d.num_attn_layers < 0 || (d.num_layers > 0 && !d.layers) ||
      (d.num_layers + d.num_attn_layers > 0 && !d.input_norm_w) ||
      (d.num_attn_layers > 0 && (!d.attn_layers || !d.kv)))
    return efail(GDN_ERR_INVALID,
                 "gdn_exec_create: NULL pool / embed / head / norm / layers / attention / kv");
  const int depth = d.num_layers + d.num_attn_layers;
  for (int l = 0; l < d.num_layers; ++l)
    if (!d.layers[l]) return efail(GDN_ERR_INVALID, "gdn_exec_create: GDN layer %d is NULL", l);
  for (int p = 0; p < depth; ++p)
    if (!d.input_norm_w[p])
      return efail(GDN_ERR_INVALID, "gdn_exec_create: norm weight of decoder layer %d is NULL", p);
  std::vector<int> stack(depth, 0);
  for (int i = 0; i < d.num_attn_layers; ++i) {
    const gdn_exec_attn_layer& a = d.attn_layers[i];
    if (a.position < 0 || a.position >= depth || (i > 0 && a.position <= d.attn_layers[i - 1].position))
      return efail(GDN_ERR_INVALID,
                   "gdn_exec_create: attention layer %d at position %d (increasing, < %d)", i,
                   a.position, depth);
    if (!a.qkv_proj || !a.o_proj || !a.q_norm_w || !a.k_norm_w)
      return efail(GDN_ERR_INVALID, "gdn_exec_create: attention layer %d has a NULL weight", i);
    stack[a.position] = -i - 1;
  }
  for (int p = 0, g = 0; p < depth; ++p)
    if (stack[p] == 0) stack[p] = g++;  // attention positions hold negative entries
  if (d.max_batch < 1 || d.max_prompt < 1)
    return efail(GDN_ERR_INVALID, "gdn_exec_create: max_batch and max_prompt must be >= 1");
  if (!(d.rms_eps >= 0.0f)) return efail(GDN_ERR_INVALID, "gdn_exec_create: rms_eps < 0");
  if (reinterpret_cast<uintptr_t>(d.embed) % 16 != 0)
    return efail(GDN_ERR_INVALID, "gdn_exec_create: embed must be 16-byte aligned");
  int32_t hidden = 0, vocab = 0;
  GDN_TRY(gdn_qlinear_dims(d.head, &hidden, &vocab));
  if (hidden > 4096) return efail(GDN_ERR_UNSUPPORTED, "gdn_exec_create: hidden %d > 4096", hidden);
  const int rows = d.max_batch > d.max_prompt ? d.max_batch : d.max_prompt;
  int Hq = 0, Hkv = 0, nqkv = 0;
  if (d.num_attn_layers > 0) {
    gdn_kv_desc kd{};
    gdn_pool_desc pd{};
    GDN_TRY(gdn_kv_describe(d.kv, &kd));
    GDN_TRY(gdn_pool_describe(d.pool, &pd));
    if (kd.num_layers < d.num_attn_layers || kd.num_slots < pd.num_slots ||
        kd.max_step_tokens < rows || kd.device != d.device)
      return efail(GDN_ERR_INVALID,
                   "gdn_exec_create: kv cache (%d layers, %d slots, %d step tokens, device %d) "
                   "does not fit %d attention layers, %d slots, %d rows, device %d",
                   kd.num_layers, kd.num_slots, kd.max_step_tokens, kd.device, d.num_attn_layers,
                   pd.num_slots, rows, d.device);
    if (d.rotary_dim < 0 || d.rotary_dim > 256 || d.rotary_dim % 2 != 0 || !(d.rope_theta > 0.0f))
      return efail(GDN_ERR_INVALID, "gdn_exec_create: rotary_dim %d / rope_theta", d.rotary_dim);
    // a prompt starts at position 0 of its slot's KV cache: the longest one
    // must fit the pages one slot can hold
    if ((int64_t)d.max_prompt > (int64_t)kd.max_pages_per_slot * 64)
      return efail(GDN_ERR_INVALID,
                   "gdn_exec_create: max_prompt %d > %lld tokens one slot's KV pages hold",
                   d.max_prompt, (long long)kd.max_pages_per_slot * 64);
    Hq = kd.num_q_heads;
    Hkv = kd.num_kv_heads;
    nqkv = 2 * Hq * 256 + 2 * Hkv * 256;
    for (int i = 0; i < d.num_attn_layers; ++i) {
      int32_t k1 = 0, n1 = 0, k2 = 0, n2 = 0;
      GDN_TRY(gdn_qlinear_dims(d.attn_layers[i].qkv_proj, &k1, &n1));
      GDN_TRY(gdn_qlinear_dims(d.attn_layers[i].o_proj, &k2, &n2));
      if (k1 != hidden || n1 != nqkv || k2 != Hq * 256 || n2 != hidden)
        return efail(GDN_ERR_INVALID,
                     "gdn_exec_create: attention layer %d projections %d->%d, %d->%d (want "
                     "%d->%d, %d->%d)",
                     i, k1, n1, k2, n2, hidden, nqkv, Hq * 256, hidden);
    }
  }
  DevScope dev(d.device);
  gdn_exec* x = new gdn_exec;
  x->pool = d.pool;
  x->layers.assign(d.layers, d.layers + d.num_layers);
  x->norm_w.assign(d.input_norm_w, d.input_norm_w + depth);
  x->stack = stack;
  for (int i = 0; i < d.num_attn_layers; ++i)
    x->attn.push_back({d.attn_layers[i].qkv_proj, d.attn_layers[i].o_proj,
                       d.attn_layers[i].q_norm_w, d.attn_layers[i].k_norm_w});
  x->kv = d.num_attn_layers > 0 ? d.kv : nullptr;
  x->rope_theta = d.rope_theta;
  x->rotary_dim = d.rotary_dim;
  x->Hq = Hq;
  x->Hkv = Hkv;
  x->nqkv = nqkv;
  x->ones.assign(d.max_batch, 1);
  x->final_norm_w = d.final_norm_w;
  x->eps = d.rms_eps;
  x->embed = d.embed;
  x->head = d.head;
  x->hidden = hidden;
  x->vocab = vocab;
  x->max_batch = d.max_batch;
  x->max_prompt = d.max_prompt;
  x->rows = rows;
  x->device = d.device;
  x->stream = static_cast<hipStream_t>(stream);
  {
    const char* g = getenv("GDN_EXEC_GRAPHS");
    x->use_graphs = !(g && g[0] == '0' && g[1] == 0);
    const char* ss = getenv("GDN_EXEC_SPLIT_SUMS");
    x->use_split_sums = !(ss && ss[0] == '0' && ss[1] == 0);
  }
  const size_t act = (size_t)x->rows * hidden * sizeof(uint16_t);
  bool ok = hipMalloc(&x->d_dec, sizeof(int32_t) * 2 * d.max_batch) == hipSuccess &&
            hipMalloc(&x->d_pre, sizeof(int32_t) * pre_words(d.max_batch, d.max_prompt)) == hipSuccess &&
            hipMalloc(&x->d_next, sizeof(int32_t) * d.max_batch) == hipSuccess &&
            hipMalloc(&x->h, act) == hipSuccess && hipMalloc(&x->hn, act) == hipSuccess &&
            hipMalloc(&x->mix, act) == hipSuccess &&
            hipMalloc(&x->xsplit, (size_t)3 * 64 * (hidden / 64 + 1) * sizeof(uint16_t)) == hipSuccess &&
            hipMalloc(&x->logits, (size_t)d.max_batch * vocab * sizeof(uint16_t)) == hipSuccess &&
            hipMalloc(&x->d_pv, sizeof(float) * d.max_batch * gdn::argmax_chunks(vocab)) == hipSuccess &&
            hipMalloc(&x->d_pi, sizeof(int) * d.max_batch * gdn::argmax_chunks(vocab)) == hipSuccess &&
            hipHostMalloc(&x->p_dec, sizeof(int32_t) * 2 * d.max_batch, 0) == hipSuccess &&
            hipHostMalloc(&x->p_pre, sizeof(int32_t) * pre_words(d.max_batch, d.max_prompt), 0) == hipSuccess &&
            hipHostMalloc(&x->p_next, sizeof(int32_t) * 2 * d.max_batch,
                          hipHostMallocMapped | hipHostMallocCoherent) == hipSuccess &&
            hipHostGetDevicePointer((void**)&x->p_next_dev, x->p_next, 0) == hipSuccess &&
            hipHostMalloc(&x->p_first, sizeof(int32_t) * d.max_batch, 0) == hipSuccess &&
            hipEventCreateWithFlags(&x->pre_copied, hipEventDisableTiming) == hipSuccess &&
            (nqkv == 0 ||
             (hipMalloc(&x->qkv, (size_t)x->rows * nqkv * sizeof(uint16_t)) == hipSuccess &&
              hipMalloc(&x->att, (size_t)x->rows * Hq * 256 * sizeof(uint16_t)) == hipSuccess));
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

gdn_status gdn_exec_prefill_batch(gdn_exec* x, int32_t nseq, const uint64_t* seq_ids,
                                  const int32_t* prompts, const int32_t* lens,
                                  uint32_t* first_tokens) {
  if (!x || !seq_ids || !prompts || !lens || !first_tokens)
    return efail(GDN_ERR_INVALID, "gdn_exec_prefill: NULL argument");
  if (nseq < 1 || nseq > x->max_batch)
    return efail(GDN_ERR_INVALID, "gdn_exec_prefill: %d sequences outside [1, %d]", nseq,
                 x->max_batch);
  int64_t total = 0;
  std::unordered_set<uint64_t> seen;
  for (int i = 0; i < nseq; ++i) {
    if (lens[i] < 1)
      return efail(GDN_ERR_INVALID, "gdn_exec_prefill: prompt %d has length %d < 1", i, lens[i]);
    if (!seen.insert(seq_ids[i]).second)
      return efail(GDN_ERR_INVALID, "gdn_exec_prefill: sequence %llu appears twice",
                   (unsigned long long)seq_ids[i]);
    total += lens[i];
  }
  if (total > x->max_prompt)
    return efail(GDN_ERR_INVALID, "gdn_exec_prefill: %lld prompt tokens > max_prompt %d",
                 (long long)total, x->max_prompt);
  for (int64_t t = 0; t < total; ++t)
    if (prompts[t] < 0 || prompts[t] >= x->vocab)
      return efail(GDN_ERR_INVALID, "gdn_exec_prefill: token %d at %lld outside [0, %d)",
                   prompts[t], (long long)t, x->vocab);
  DevScope dev(x->device);
  x->chain_B = 0;  // the next decode step takes its tokens from the host
  // The pinned block is free once the previous prefill's copy has run (a
  // prefill that failed after queueing it may not have waited).
  HIP_TRY(hipEventSynchronize(x->pre_copied), "gdn_exec_prefill");
  if (x->kv) {
    // the KV pages the prompts need against those free plus those the
    // restarting (known) sequences give back, and each prompt against one
    // slot's page table: checked before anything changes
    gdn_kv_desc kd{};
    GDN_TRY(gdn_kv_describe(x->kv, &kd));
    int32_t free_pages = 0;
    GDN_TRY(gdn_kv_free_pages(x->kv, &free_pages));
    int64_t avail = free_pages, need = 0;
    for (int i = 0; i < nseq; ++i) {
      if ((int64_t)lens[i] > (int64_t)kd.max_pages_per_slot * 64)
        return efail(GDN_ERR_INVALID, "gdn_exec_prefill: prompt %d of %d tokens > %lld per slot",
                     i, lens[i], (long long)kd.max_pages_per_slot * 64);
      need += (lens[i] + 63) / 64;
      auto it = x->slot_of.find(seq_ids[i]);
      if (it != x->slot_of.end()) {
        int64_t len = 0;
        GDN_TRY(gdn_kv_length(x->kv, it->second, &len));
        avail += (len + 63) / 64;
      }
    }
    if (need > avail)
      return efail(GDN_ERR_OOM, "gdn_exec_prefill: %lld KV pages needed, %lld available",
                   (long long)need, (long long)avail);
  }
  // admit: a fresh sequence gets a free slot, a known one starts over in its
  // own; a call that runs out of slots gives back the ones it took
  int32_t* slots = x->p_pre;
  std::vector<int> fresh;
  for (int i = 0; i < nseq; ++i) {
    auto it = x->slot_of.find(seq_ids[i]);
    if (it != x->slot_of.end()) {
      slots[i] = it->second;
      continue;
    }
    if (gdn_slot_alloc(x->pool, &slots[i]) != GDN_OK) {
      for (int k : fresh) {
        (void)gdn_slot_free(x->pool, slots[k]);
        x->slot_of.erase(seq_ids[k]);
      }
      return efail(GDN_ERR_SLOTS, "gdn_exec_prefill: no free slot for sequence %llu",
                   (unsigned long long)seq_ids[i]);
    }
    x->slot_of.emplace(seq_ids[i], slots[i]);
    fresh.push_back(i);
  }
  // From here on a failure leaves the call's sequences without a usable
  // state (a known sequence has given back its KV pages, and its GDN state may
  // be zeroed or half updated): every sequence of the call is retired (slot and
  // pages freed, id forgotten), and the caller prefills it again.
  auto retire_call = [&](gdn_status st) {
    for (int i = 0; i < nseq; ++i) {
      auto it = x->slot_of.find(seq_ids[i]);
      if (it == x->slot_of.end()) continue;
      (void)gdn_slot_free(x->pool, it->second);
      if (x->kv) (void)gdn_kv_release(x->kv, it->second);
      x->slot_of.erase(it);
    }
    return st;
  };
#define GDN_TRY_RETIRE(expr)                  \
  do {                                        \
    gdn_status st_ = (expr);                  \
    if (st_ != GDN_OK) return retire_call(st_); \
  } while (0)
#define HIP_TRY_RETIRE(expr, what)                            \
  do {                                                        \
    hipError_t e_ = (expr);                                   \
    if (e_ != hipSuccess) return retire_call(hfail(e_, what)); \
  } while (0)
  if (x->kv) {
    // every prompt starts at position 0 of its slot's KV cache
    for (int i = 0; i < nseq; ++i) GDN_TRY_RETIRE(gdn_kv_release(x->kv, slots[i]));
    GDN_TRY_RETIRE(gdn_kv_step(x->kv, nseq, slots, lens, x->stream));
  }
  int32_t* cu = x->p_pre + nseq;
  int32_t* last = cu + nseq + 1;
  int32_t* toks = last + nseq;
  cu[0] = 0;
  for (int i = 0; i < nseq; ++i) {
    cu[i + 1] = cu[i] + lens[i];
    last[i] = cu[i + 1] - 1;
  }
  for (int64_t t = 0; t < total; ++t) toks[t] = prompts[t];
  const int32_t* d_cu = x->d_pre + nseq;
  const int32_t* d_last = d_cu + nseq + 1;
  const int32_t* d_toks = d_last + nseq;
  HIP_TRY_RETIRE(hipMemcpyAsync(x->d_pre, x->p_pre,
                                sizeof(int32_t) * (3 * (size_t)nseq + 1 + total),
                                hipMemcpyHostToDevice, x->stream),
                 "prompt copy");
  HIP_TRY_RETIRE(hipEventRecord(x->pre_copied, x->stream), "prompt copy event");
  GDN_TRY_RETIRE(gdn_slots_zero(x->pool, GDN_ALL_LAYERS, x->d_pre, nseq, x->stream));
  const int n = (int)total;
  GDN_TRY_RETIRE(run_layers(x, n, true, d_toks, nseq));
  // final residual add + norm of every row, then each prompt's last row
  HIP_TRY_RETIRE(gdn::launch_add_norm(x->h, x->stack.empty() ? nullptr : x->mix,
                                      x->stack.empty() ? nullptr : &x->pend, n, x->hidden,
                                      x->final_norm_w, x->eps, x->hn, x->stream),
                 "final norm");
  x->pend = gdn::QPartial{};
  HIP_TRY_RETIRE(gdn::launch_gather_rows(x->hn, d_last, nseq, x->hidden, x->mix, x->stream),
                 "last rows");
  GDN_TRY_RETIRE(
      gdn_qlinear_forward(x->head, x->mix, x->hidden, nseq, x->logits, x->vocab, x->stream));
  HIP_TRY_RETIRE(gdn::launch_argmax(x->logits, x->vocab, nseq, x->vocab, x->d_pv, x->d_pi,
                                    x->d_next, nullptr, x->stream),
                 "argmax");
  HIP_TRY_RETIRE(hipMemcpyAsync(x->p_first, x->d_next, sizeof(int32_t) * nseq,
                                hipMemcpyDeviceToHost, x->stream),
                 "token copy");
  x->logits_rows = nseq;
  HIP_TRY_RETIRE(hipStreamSynchronize(x->stream), "gdn_exec_prefill sync");
#undef GDN_TRY_RETIRE
#undef HIP_TRY_RETIRE
  for (int i = 0; i < nseq; ++i) first_tokens[i] = (uint32_t)x->p_first[i];
  return GDN_OK;
}

gdn_status gdn_exec_prefill(gdn_exec* x, uint64_t seq_id, const int32_t* prompt, int32_t len,
                            uint32_t* first_token) {
  return gdn_exec_prefill_batch(x, 1, &seq_id, prompt, &len, first_token);
}

gdn_status gdn_exec_submit_batch(gdn_exec* x, const uint64_t* seq_ids, const uint32_t* tokens,
                                 int32_t B) {
  if (!x) return efail(GDN_ERR_INVALID, "gdn_exec_submit_batch: NULL executor");
  if (x->pend_n > 0)
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
  }
  for (int b = 0; b < B; ++b) {
    x->p_dec[b] = x->slot_of[seq_ids[b]];
    x->p_dec[x->max_batch + b] = (int32_t)tokens[b];
  }
  DevScope dev(x->device);
  x->chain_B = 0;
  // plan the attention layers' KV step first: it fails (changing nothing)
  // when the cache is out of pages, before any device work is queued
  if (x->kv) GDN_TRY(gdn_kv_step(x->kv, B, x->p_dec, x->ones.data(), x->stream));
  HIP_TRY(hipMemcpyAsync(x->d_dec, x->p_dec, sizeof(int32_t) * 2 * x->max_batch,
                         hipMemcpyHostToDevice, x->stream),
          "batch copy");
  return queue_step(x, B);
}

gdn_status gdn_exec_submit_next(gdn_exec* x, int32_t B) {
  if (!x) return efail(GDN_ERR_INVALID, "gdn_exec_submit_next: NULL executor");
  if (x->chain_B == 0)
    return efail(GDN_ERR_INVALID,
                 "gdn_exec_submit_next: no decode step to follow (none submitted since the "
                 "last prefill or release)");
  if (B != x->chain_B)
    return efail(GDN_ERR_INVALID, "gdn_exec_submit_next: B = %d, the step it follows has %d", B,
                 x->chain_B);
  if (x->pend_n == 2)
    return efail(GDN_ERR_INVALID, "gdn_exec_submit_next: two submitted steps are not collected yet");
  DevScope dev(x->device);
  // the same slots (p_dec is written only by gdn_exec_submit_batch)
  if (x->kv) GDN_TRY(gdn_kv_step(x->kv, B, x->p_dec, x->ones.data(), x->stream));
  return queue_step(x, B);
}

// Time collect polls the pick slot with a pause between polls before it starts
// to yield the core between them: ten decode steps and more. (Yielding from
// the first step's worth of polls on made host-fed steps of ~2.2 ms take up to
// 3.4 ms: a yielding thread can lose its core near the end of the wait.)
constexpr auto kCollectSpinTime = std::chrono::milliseconds(20);

gdn_status gdn_exec_collect_batch(gdn_exec* x, uint32_t* next_tokens, int32_t B) {
  if (!x || !next_tokens) return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: NULL argument");
  if (x->pend_n == 0) return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: nothing submitted");
  const int e = x->pend_head;
  if (B != x->pend_B[e])
    return efail(GDN_ERR_INVALID, "gdn_exec_collect_batch: B = %d, submitted %d", B,
                 x->pend_B[e]);
  x->pend_head ^= 1;
  --x->pend_n;
  // The greedy pick writes the step's tokens (>= 0) into the pinned slot, the
  // step's last device work. Poll it, with a pause instruction between polls;
  // after kCollectSpinTime of polling give the core up between polls (yield).
  // Every 1024 polls look at the clock and ask the stream for an error, and a
  // stream that has drained with picks missing is one.
  volatile const int32_t* picks = x->p_next + (size_t)e * x->max_batch;
  auto landed = [&]() {
    for (int b = 0; b < B; ++b)
      if (picks[b] < 0) return false;
    return true;
  };
  const auto t0 = std::chrono::steady_clock::now();
  bool yielding = false;
  for (uint64_t spin = 1; !landed(); ++spin) {
    if (yielding)
      std::this_thread::yield();
    else
      __builtin_ia32_pause();
    if (spin % 1024 != 0) continue;
    yielding = yielding || std::chrono::steady_clock::now() - t0 > kCollectSpinTime;
    const hipError_t q = hipStreamQuery(x->stream);
    if (q == hipErrorNotReady) continue;
    if (q != hipSuccess) return hfail(q, "gdn_exec_collect_batch");
    if (!landed())
      return efail(GDN_ERR_HIP, "gdn_exec_collect_batch: the step ended without its picks");
    break;
  }
  for (int b = 0; b < B; ++b) next_tokens[b] = (uint32_t)picks[b];
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
  x->chain_B = 0;
  GDN_TRY(gdn_slot_free(x->pool, it->second));
  if (x->kv) GDN_TRY(gdn_kv_release(x->kv, it->second));
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
