// gdn_kv.cpp -- paged KV cache of the attention layers and the attention
// step entry (gdn_kv_*, gdn_attn_forward).
//
// The reference keeps one growing [1, Hkv, len, 256] key and value array per
// sequence and layer and concatenates every new token onto it
// (qwen3_5.rs:419-424); batching pads them all to the longest
// (mlx_executor.rs:57-88). Here the cache is pages of 64 tokens, one page id
// covering the same positions in every layer, handed out by a host free list;
// a sequence's page table maps position / 64 to its pages. A step first
// plans the tokens it appends (gdn_kv_step: per token its sequence slot,
// position and page, and the attention schedule, staged to the device once
// for all layers), then each attention layer runs gdn_attn_forward on the
// same packed tokens.
//
// The schedule: the step's tokens form groups of up to 16 / G consecutive
// tokens of one sequence (G query heads per kv head: a group's (token, head)
// pairs fill the 16 columns of an MFMA tile); each (group, kv head) segment
// is its keys, cut into chunks of 384 keys at fixed points. All segments'
// chunks, in order, go to P one-wave workers in equal runs of kpw, P up to
// max_workers (default below). Every chunk writes one partial and the
// combine kernel merges a segment's partials in order, so a token's result
// does not depend on the rest of the step.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <climits>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <unordered_set>
#include <vector>

#include "gdn.h"
#include "gdn_common.h"

namespace {

gdn_status kfail(gdn_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  return gdn::set_error(code, buf);
}

gdn_status khip(hipError_t e, const char* what) {
  return kfail(GDN_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

constexpr int kPageTokens = 64;
constexpr int kHeadDim = 256;
// Workers per step: a step whose key blocks are each read about once (decode)
// streams from HBM and runs best near one wave per SIMD (256 CUs x 4); one
// that re-reads them from cache (a prompt's token groups share its keys)
// wants the two resident waves per SIMD the block kernel's registers allow.
constexpr int kStreamWorkers = 1536;  // equal runs of chunks: 768 .. 1536 workers
constexpr int kReuseWorkers = 2048;

// int32 words of the step metadata for up to T tokens and P workers
size_t meta_words(int T, int Hkv, int P) { return (size_t)T * (5 + 4 + 4 * (size_t)Hkv) + P; }

int max_workers(const gdn_kv_desc& d) { return d.max_workers > 0 ? d.max_workers : kReuseWorkers; }

struct Dev {
  int prev = -1;
  explicit Dev(int dev) {
    if (hipGetDevice(&prev) == hipSuccess && prev != dev) (void)hipSetDevice(dev);
  }
  ~Dev() {
    int cur = -1;
    if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
  }
};

}  // namespace

struct gdn_kv {
  gdn_kv_desc d{};
  std::vector<uint16_t*> pages;  // per layer [num_pages][2][Hkv][64][256] bf16
  int32_t* ptab = nullptr;       // [num_slots][max_pages_per_slot]
  std::vector<int32_t> free_pages;
  std::vector<int64_t> len;                  // tokens cached per slot
  std::vector<std::vector<int32_t>> owned;   // pages per slot, in position order
  // step metadata: [3][T] slot, position, page; [2][T] group, first column;
  // grp [NG][4]; seg [NG * Hkv][4]; wseg [P]
  int32_t* d_meta = nullptr;
  int32_t* p_meta = nullptr;     // pinned staging
  hipEvent_t meta_copied = nullptr;
  void* workspace = nullptr;
  size_t ws_bytes = 0;
  // the planned step
  int T = 0, NG = 0, P = 0, NC = 0, kpw = 0;
  bool stream_keys = false;
  bool planned = false;
};

namespace {

void kv_release_all(gdn_kv* kv) {
  if (!kv) return;
  for (uint16_t* p : kv->pages)
    if (p) (void)hipFree(p);
  if (kv->ptab) (void)hipFree(kv->ptab);
  if (kv->d_meta) (void)hipFree(kv->d_meta);
  if (kv->p_meta) (void)hipHostFree(kv->p_meta);
  if (kv->meta_copied) (void)hipEventDestroy(kv->meta_copied);
  if (kv->workspace) (void)hipFree(kv->workspace);
  delete kv;
}

}  // namespace

extern "C" {

gdn_status gdn_kv_create(const gdn_kv_desc* desc, gdn_kv** out) {
  if (!desc || !out) return kfail(GDN_ERR_INVALID, "gdn_kv_create: desc/out is NULL");
  *out = nullptr;
  const gdn_kv_desc& d = *desc;
  if (d.num_layers < 1 || d.num_slots < 1 || d.num_pages < 1 || d.max_pages_per_slot < 1 ||
      d.max_step_tokens < 1 || d.num_kv_heads < 1 || d.num_q_heads < 1)
    return kfail(GDN_ERR_INVALID, "gdn_kv_create: sizes must be >= 1");
  if (d.head_dim != kHeadDim)
    return kfail(GDN_ERR_UNSUPPORTED, "gdn_kv_create: head_dim %d (compiled for 256)", d.head_dim);
  if (d.num_q_heads % d.num_kv_heads != 0 ||
      (d.num_q_heads / d.num_kv_heads != 4 && d.num_q_heads / d.num_kv_heads != 8))
    return kfail(GDN_ERR_UNSUPPORTED, "gdn_kv_create: %d query heads per kv head (4 or 8 supported)",
                 d.num_q_heads / d.num_kv_heads);
  if (d.max_workers < 0 || d.max_workers > 65536)
    return kfail(GDN_ERR_INVALID, "gdn_kv_create: max_workers %d outside [0, 65536]", d.max_workers);
  if ((int64_t)d.max_pages_per_slot * kPageTokens > (int64_t)1 << 30)
    return kfail(GDN_ERR_INVALID, "gdn_kv_create: max_pages_per_slot too large");
  Dev dev(d.device);
  gdn_kv* kv = new gdn_kv;
  kv->d = d;

  const size_t page_bytes = (size_t)2 * d.num_kv_heads * kPageTokens * kHeadDim * 2;
  bool ok = true;
  for (int l = 0; l < d.num_layers && ok; ++l) {
    uint16_t* p = nullptr;
    ok = hipMalloc(&p, page_bytes * d.num_pages) == hipSuccess;
    kv->pages.push_back(p);
  }
  const size_t mwords = meta_words(d.max_step_tokens, d.num_kv_heads, max_workers(d));
  ok = ok && hipMalloc(&kv->ptab, sizeof(int32_t) * d.num_slots * d.max_pages_per_slot) == hipSuccess &&
       hipMalloc(&kv->d_meta, sizeof(int32_t) * mwords) == hipSuccess &&
       hipHostMalloc(&kv->p_meta, sizeof(int32_t) * mwords, 0) == hipSuccess &&
       hipEventCreateWithFlags(&kv->meta_copied, hipEventDisableTiming) == hipSuccess;
  if (!ok) {
    (void)hipGetLastError();
    kv_release_all(kv);
    return kfail(GDN_ERR_OOM, "gdn_kv_create: %d layers x %d pages of %zu bytes", d.num_layers,
                 d.num_pages, page_bytes);
  }
  // The attention workspace of any decode step (one token per sequence),
  // sized once: n <= min(max_step_tokens, num_slots) sequences, each
  // segment's keys cut into chunks of C blocks. Sequences hold distinct
  // pages, so their blocks add up to at most 4 per page in the cache plus
  // one partial block each: chunks <= Hkv (n + (4 num_pages + 2 n) / C + 2).
  // A step with prompts (several tokens of one sequence, each group of them
  // reading the shared prefix) can need more and then grows it.
  {
    const int64_t n = d.max_step_tokens < d.num_slots ? d.max_step_tokens : d.num_slots;
    const int64_t chunks =
        (int64_t)d.num_kv_heads * (n + (4 * (int64_t)d.num_pages + 2 * n) / gdn::attn_chunk_blocks() + 2);
    const size_t ws = gdn::attn_workspace_bytes((int)n, d.num_q_heads, chunks);
    if (hipMalloc(&kv->workspace, ws) != hipSuccess) {
      (void)hipGetLastError();
      kv_release_all(kv);
      return kfail(GDN_ERR_OOM, "gdn_kv_create: attention workspace of %zu bytes", ws);
    }
    kv->ws_bytes = ws;
  }
  kv->free_pages.resize(d.num_pages);
  for (int i = 0; i < d.num_pages; ++i) kv->free_pages[i] = d.num_pages - 1 - i;  // pop lowest first
  kv->len.assign(d.num_slots, 0);
  kv->owned.resize(d.num_slots);
  *out = kv;
  return GDN_OK;
}

gdn_status gdn_kv_destroy(gdn_kv* kv) {
  if (!kv) return GDN_OK;
  Dev dev(kv->d.device);
  kv_release_all(kv);
  return GDN_OK;
}

gdn_status gdn_kv_describe(const gdn_kv* kv, gdn_kv_desc* desc) {
  if (!kv || !desc) return kfail(GDN_ERR_INVALID, "gdn_kv_describe: NULL argument");
  *desc = kv->d;
  return GDN_OK;
}

gdn_status gdn_kv_release(gdn_kv* kv, int32_t slot) {
  if (!kv) return kfail(GDN_ERR_INVALID, "gdn_kv_release: NULL cache");
  if (slot < 0 || slot >= kv->d.num_slots)
    return kfail(GDN_ERR_INVALID, "gdn_kv_release: slot %d outside [0, %d)", slot, kv->d.num_slots);
  for (int32_t p : kv->owned[slot]) kv->free_pages.push_back(p);
  kv->owned[slot].clear();
  kv->len[slot] = 0;
  return GDN_OK;
}

gdn_status gdn_kv_length(const gdn_kv* kv, int32_t slot, int64_t* len) {
  if (!kv || !len) return kfail(GDN_ERR_INVALID, "gdn_kv_length: NULL argument");
  if (slot < 0 || slot >= kv->d.num_slots)
    return kfail(GDN_ERR_INVALID, "gdn_kv_length: slot %d outside [0, %d)", slot, kv->d.num_slots);
  *len = kv->len[slot];
  return GDN_OK;
}

gdn_status gdn_kv_free_pages(const gdn_kv* kv, int32_t* count) {
  if (!kv || !count) return kfail(GDN_ERR_INVALID, "gdn_kv_free_pages: NULL argument");
  *count = (int32_t)kv->free_pages.size();
  return GDN_OK;
}

gdn_status gdn_kv_step(gdn_kv* kv, int32_t n, const int32_t* slots, const int32_t* ntok,
                       void* stream) {
  if (!kv || !slots || !ntok) return kfail(GDN_ERR_INVALID, "gdn_kv_step: NULL argument");
  const gdn_kv_desc& d = kv->d;
  if (n < 1) return kfail(GDN_ERR_INVALID, "gdn_kv_step: n = %d < 1", n);
  int64_t T = 0;
  std::unordered_set<int32_t> seen;
  for (int i = 0; i < n; ++i) {
    if (slots[i] < 0 || slots[i] >= d.num_slots)
      return kfail(GDN_ERR_INVALID, "gdn_kv_step: slot %d outside [0, %d)", slots[i], d.num_slots);
    if (!seen.insert(slots[i]).second)
      return kfail(GDN_ERR_INVALID, "gdn_kv_step: slot %d appears twice", slots[i]);
    if (ntok[i] < 1) return kfail(GDN_ERR_INVALID, "gdn_kv_step: %d new tokens < 1", ntok[i]);
    if (kv->len[slots[i]] + ntok[i] > (int64_t)d.max_pages_per_slot * kPageTokens)
      return kfail(GDN_ERR_INVALID, "gdn_kv_step: slot %d would hold %lld tokens > %lld",
                   slots[i], (long long)(kv->len[slots[i]] + ntok[i]),
                   (long long)d.max_pages_per_slot * kPageTokens);
    T += ntok[i];
  }
  if (T > d.max_step_tokens)
    return kfail(GDN_ERR_INVALID, "gdn_kv_step: %lld tokens > max_step_tokens %d", (long long)T,
                 d.max_step_tokens);
  int64_t need = 0;
  for (int i = 0; i < n; ++i) {
    const int64_t have = (int64_t)kv->owned[slots[i]].size();
    const int64_t want = (kv->len[slots[i]] + ntok[i] + kPageTokens - 1) / kPageTokens;
    need += want > have ? want - have : 0;
  }
  if (need > (int64_t)kv->free_pages.size())
    return kfail(GDN_ERR_OOM, "gdn_kv_step: %lld new pages needed, %zu free", (long long)need,
                 kv->free_pages.size());
  Dev dev(d.device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  // the attention schedule and workspace for this step, sized before any
  // state changes
  const int G = d.num_q_heads / d.num_kv_heads, Hkv = d.num_kv_heads;
  const int tpg = 16 / G;
  struct Group {
    int32_t t0, ntok, pos0, slot;
  };
  std::vector<Group> groups;
  {
    int32_t t0 = 0;
    for (int i = 0; i < n; ++i) {
      for (int32_t k = 0; k < ntok[i]; k += tpg) {
        const int32_t nt = ntok[i] - k < tpg ? ntok[i] - k : tpg;
        groups.push_back({t0 + k, nt, (int32_t)(kv->len[slots[i]] + k), slots[i]});
      }
      t0 += ntok[i];
    }
  }
  const int NG = (int)groups.size(), NS = NG * Hkv;
  // each segment's keys in chunks of C 16-key blocks, numbered in segment order
  const int C = gdn::attn_chunk_blocks();
  std::vector<int64_t> cs0(NS + 1);
  cs0[0] = 0;
  int64_t W = 0, distinct = 0;
  for (int gi = 0; gi < NG; ++gi) {
    const int64_t nblk = ((int64_t)groups[gi].pos0 + groups[gi].ntok + 15) / 16;
    for (int j = 0; j < Hkv; ++j) cs0[gi * Hkv + j + 1] = cs0[gi * Hkv + j] + (nblk + C - 1) / C;
    W += nblk * Hkv;
    // distinct blocks: each sequence's keys once per kv head (its last group's)
    if (gi + 1 == NG || groups[gi + 1].slot != groups[gi].slot) distinct += nblk * Hkv;
  }
  const int64_t NC = cs0[NS];
  if (NC > INT32_MAX / 2) return kfail(GDN_ERR_INVALID, "gdn_kv_step: %lld key chunks", (long long)NC);
  const bool stream_keys = W < 2 * distinct;
  const int pmax = d.max_workers > 0 ? d.max_workers : (stream_keys ? kStreamWorkers : kReuseWorkers);
  // equal runs of kpw chunks: kpw = ceil(NC / pmax), P = ceil(NC / kpw) <= pmax
  const int kpw = (int)((NC + pmax - 1) / pmax);
  const int P = (int)((NC + kpw - 1) / kpw);
  std::vector<int32_t> wseg(P);
  {
    int sg = 0;
    for (int ww = 0; ww < P; ++ww) {
      while (cs0[sg + 1] <= (int64_t)ww * kpw) ++sg;
      wseg[ww] = sg;
    }
  }
  const int64_t pieces = NC;
  const size_t ws = gdn::attn_workspace_bytes((int)T, d.num_q_heads, pieces);
  hipError_t e;
  if (ws > kv->ws_bytes) {
    if (kv->workspace) {
      if ((e = hipStreamSynchronize(s)) != hipSuccess) return khip(e, "workspace grow sync");
      (void)hipFree(kv->workspace);
      kv->workspace = nullptr;
      kv->ws_bytes = 0;
    }
    if (hipMalloc(&kv->workspace, ws) != hipSuccess) {
      (void)hipGetLastError();
      kv->planned = false;
      return kfail(GDN_ERR_OOM, "gdn_kv_step: attention workspace of %zu bytes", ws);
    }
    kv->ws_bytes = ws;
  }
  // the pinned block is free once the previous step's copy has run
  if ((e = hipEventSynchronize(kv->meta_copied)) != hipSuccess) return khip(e, "gdn_kv_step");
  int32_t* m_slot = kv->p_meta;
  int32_t* m_pos = kv->p_meta + T;
  int32_t* m_page = kv->p_meta + 2 * T;
  int32_t* m_tokseg = kv->p_meta + 3 * T;
  int32_t* m_grp = kv->p_meta + 5 * T;
  int32_t* m_seg = m_grp + 4 * NG;
  int32_t* m_wseg = m_seg + 4 * NS;
  for (int gi = 0; gi < NG; ++gi) {
    const Group& g = groups[gi];
    m_grp[4 * gi] = g.t0;
    m_grp[4 * gi + 1] = g.ntok;
    m_grp[4 * gi + 2] = g.pos0;
    m_grp[4 * gi + 3] = g.slot;
    for (int k = 0; k < g.ntok; ++k) {
      m_tokseg[g.t0 + k] = gi;
      m_tokseg[T + g.t0 + k] = k * G;
    }
  }
  for (int sg = 0; sg < NS; ++sg) {
    m_seg[4 * sg] = (int32_t)cs0[sg];
    m_seg[4 * sg + 1] = (int32_t)(cs0[sg + 1] - cs0[sg]);
    m_seg[4 * sg + 2] = 0;
    m_seg[4 * sg + 3] = 0;
  }
  for (int ww = 0; ww < P; ++ww) m_wseg[ww] = wseg[ww];
  const size_t words = (size_t)5 * T + 4 * (size_t)NG + 4 * (size_t)NS + P;
  int64_t t = 0;
  for (int i = 0; i < n; ++i) {
    const int32_t sl = slots[i];
    for (int k = 0; k < ntok[i]; ++k, ++t) {
      const int64_t pos = kv->len[sl] + k;
      if (pos / kPageTokens >= (int64_t)kv->owned[sl].size()) {
        kv->owned[sl].push_back(kv->free_pages.back());
        kv->free_pages.pop_back();
      }
      m_slot[t] = sl;
      m_pos[t] = (int32_t)pos;
      m_page[t] = kv->owned[sl][pos / kPageTokens];
    }
    kv->len[sl] += ntok[i];
  }
  if ((e = hipMemcpyAsync(kv->d_meta, kv->p_meta, sizeof(int32_t) * words, hipMemcpyHostToDevice,
                          s)) != hipSuccess ||
      (e = hipEventRecord(kv->meta_copied, s)) != hipSuccess) {
    kv->planned = false;
    return khip(e, "gdn_kv_step copy");
  }
  kv->T = (int)T;
  kv->NG = NG;
  kv->P = P;
  kv->NC = (int)NC;
  kv->kpw = kpw;
  kv->stream_keys = stream_keys;
  kv->planned = true;
  return GDN_OK;
}

gdn_status gdn_attn_forward(gdn_kv* kv, int32_t layer, const uint16_t* q_full, int64_t q_stride,
                            const uint16_t* k, int64_t k_stride, const uint16_t* v,
                            int64_t v_stride, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                            float norm_eps, float rope_theta, int32_t rotary_dim, uint16_t* out,
                            int64_t out_stride, void* stream) {
  if (!kv) return kfail(GDN_ERR_INVALID, "gdn_attn_forward: NULL cache");
  const gdn_kv_desc& d = kv->d;
  if (layer < 0 || layer >= d.num_layers)
    return kfail(GDN_ERR_INVALID, "gdn_attn_forward: layer %d outside [0, %d)", layer, d.num_layers);
  if (!kv->planned) return kfail(GDN_ERR_INVALID, "gdn_attn_forward: no step planned (gdn_kv_step)");
  if (!q_full || !k || !v || !q_norm_w || !k_norm_w || !out)
    return kfail(GDN_ERR_INVALID, "gdn_attn_forward: NULL tensor pointer");
  if (q_stride < 2LL * d.num_q_heads * kHeadDim || k_stride < (int64_t)d.num_kv_heads * kHeadDim ||
      v_stride < (int64_t)d.num_kv_heads * kHeadDim || out_stride < (int64_t)d.num_q_heads * kHeadDim)
    return kfail(GDN_ERR_INVALID, "gdn_attn_forward: row strides below the head widths");
  if (rotary_dim < 0 || rotary_dim > kHeadDim || rotary_dim % 2 != 0)
    return kfail(GDN_ERR_INVALID, "gdn_attn_forward: rotary_dim %d", rotary_dim);
  if (!(norm_eps >= 0.0f) || !(rope_theta > 0.0f))
    return kfail(GDN_ERR_INVALID, "gdn_attn_forward: norm_eps / rope_theta");
  Dev dev(d.device);
  gdn::AttnArgs a{};
  a.T = kv->T;
  a.Hq = d.num_q_heads;
  a.Hkv = d.num_kv_heads;
  a.P = kv->P;
  a.NC = kv->NC;
  a.kpw = kv->kpw;
  a.stream_keys = kv->stream_keys;
  a.max_pages = d.max_pages_per_slot;
  a.rot_dim = rotary_dim;
  a.eps = norm_eps;
  a.log2_base = (float)std::log2((double)rope_theta);
  a.q_full = q_full;
  a.qs = q_stride;
  a.k = k;
  a.ks = k_stride;
  a.v = v;
  a.vs = v_stride;
  a.q_norm_w = q_norm_w;
  a.k_norm_w = k_norm_w;
  a.meta = kv->d_meta;
  a.tokseg = kv->d_meta + 3 * (size_t)kv->T;
  a.grp = kv->d_meta + 5 * (size_t)kv->T;
  a.seg = a.grp + 4 * (size_t)kv->NG;
  a.wseg = a.seg + 4 * (size_t)kv->NG * d.num_kv_heads;
  a.ptab = kv->ptab;
  a.pages = kv->pages[layer];
  a.out = out;
  a.os = out_stride;
  a.workspace = kv->workspace;
  a.stream = static_cast<hipStream_t>(stream);
  hipError_t e = gdn::launch_attn(a);
  if (e != hipSuccess) return khip(e, "gdn_attn_forward launch");
  return GDN_OK;
}

gdn_status gdn_kv_read(gdn_kv* kv, int32_t layer, int32_t slot, uint16_t* k_out, uint16_t* v_out,
                       void* stream) {
  if (!kv || (!k_out && !v_out)) return kfail(GDN_ERR_INVALID, "gdn_kv_read: NULL argument");
  const gdn_kv_desc& d = kv->d;
  if (layer < 0 || layer >= d.num_layers || slot < 0 || slot >= d.num_slots)
    return kfail(GDN_ERR_INVALID, "gdn_kv_read: layer %d / slot %d out of range", layer, slot);
  Dev dev(d.device);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t L = kv->len[slot];
  hipError_t e = gdn::launch_kv_gather(kv->pages[layer],
                                       kv->ptab + (size_t)slot * d.max_pages_per_slot,
                                       d.num_kv_heads, L, k_out, v_out, s);
  if (e != hipSuccess) return khip(e, "gdn_kv_read");
  return GDN_OK;
}

}  // extern "C"
