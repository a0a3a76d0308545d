// Host-code test of libgdn under AddressSanitizer / UBSan: the pool's slot
// allocator, argument checks, the debug slot-list check, the KV cache's page
// planner and accounting, and the executor's admission, batching, error and
// rollback paths, run against the runtime stand-in in fake_hip.cpp (no GPU;
// kernels compute nothing). Exits 0 and prints "ALL OK" when every check holds.
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "gdn.h"

namespace gdn_fake {
extern bool fail_embed;  // fake_hip.cpp: the next embedding launches fail
extern bool capture;     // fake_hip.cpp: stream capture makes (empty) graphs
extern bool split;       // fake_hip.cpp: prefill calls take the split path
extern int graphs_live, graphs_destroyed, graphs_made;
}

static int g_checks = 0;
#define CHECK(cond)                                                                \
  do {                                                                             \
    ++g_checks;                                                                    \
    if (!(cond)) {                                                                 \
      std::fprintf(stderr, "FAILED %s:%d: %s (last error: %s)\n", __FILE__, __LINE__, \
                   #cond, gdn_last_error());                                       \
      return 1;                                                                    \
    }                                                                              \
  } while (0)

template <typename T>
static T* dev_alloc(std::vector<std::vector<char>>& keep, size_t n) {
  keep.emplace_back(n * sizeof(T) + 16, 0);
  char* p = keep.back().data();
  return reinterpret_cast<T*>(p + ((16 - reinterpret_cast<uintptr_t>(p) % 16) % 16));
}

static gdn_qlinear* make_qlinear(std::vector<std::vector<char>>& keep, int K,
                                 std::vector<int32_t> rows) {
  std::vector<const uint32_t*> w;
  std::vector<const uint16_t*> s, b;
  for (int32_t n : rows) {
    w.push_back(dev_alloc<uint32_t>(keep, (size_t)n * K / 8));
    s.push_back(dev_alloc<uint16_t>(keep, (size_t)n * K / 64));
    b.push_back(dev_alloc<uint16_t>(keep, (size_t)n * K / 64));
  }
  gdn_qlinear* q = nullptr;
  if (gdn_qlinear_create(K, (int)rows.size(), rows.data(), w.data(), s.data(), b.data(), 64, 4, 0,
                         nullptr, &q) != GDN_OK)
    return nullptr;
  return q;
}

static int test_pool() {
  gdn_pool_desc d{2, 8, 16, 32, 128, 128, 4, 0};
  gdn_pool* pool = nullptr;
  CHECK(gdn_pool_create(&d, &pool) == GDN_OK && pool);
  int32_t s = -1, n = 0;
  for (int i = 0; i < 8; ++i) CHECK(gdn_slot_alloc(pool, &s) == GDN_OK && s == i);
  CHECK(gdn_slot_alloc(pool, &s) == GDN_ERR_SLOTS);
  CHECK(gdn_slot_free(pool, 5) == GDN_OK);
  CHECK(gdn_slot_free(pool, 5) == GDN_ERR_SLOTS);
  CHECK(gdn_slot_free(pool, 8) == GDN_ERR_SLOTS);
  CHECK(gdn_slots_in_use(pool, &n) == GDN_OK && n == 7);
  CHECK(gdn_slot_alloc(pool, &s) == GDN_OK && s == 5);
  std::vector<std::vector<char>> keep;
  int32_t* ids = dev_alloc<int32_t>(keep, 4);
  CHECK(gdn_slots_zero(pool, GDN_ALL_LAYERS, ids, -1, nullptr) == GDN_ERR_INVALID);
  CHECK(gdn_slots_zero(pool, GDN_ALL_LAYERS, ids, 0, nullptr) == GDN_OK);
  CHECK(gdn_slots_zero(pool, 2, ids, 1, nullptr) == GDN_ERR_INVALID);
  CHECK(gdn_slots_read(pool, 0, nullptr, 1, nullptr, nullptr, nullptr) == GDN_ERR_INVALID);
  // decode arguments and the debug slot-list check (this build defines GDN_DEBUG_SLOTS)
  const int D = 8192;
  uint16_t* x = dev_alloc<uint16_t>(keep, 4 * D);
  uint16_t* ab = dev_alloc<uint16_t>(keep, 4 * 64);
  float* al = dev_alloc<float>(keep, 32);
  float* dt = dev_alloc<float>(keep, 32);
  uint16_t* cw = dev_alloc<uint16_t>(keep, (size_t)D * 4);
  uint16_t* y = dev_alloc<uint16_t>(keep, 4 * 32 * 128);
  ids[0] = 3; ids[1] = 1; ids[2] = 6; ids[3] = 0;
  CHECK(gdn_decode(pool, 0, ids, 4, x, ab, al, dt, cw, y, nullptr) == GDN_OK);
  CHECK(gdn_decode(pool, 0, ids, 9, x, ab, al, dt, cw, y, nullptr) == GDN_ERR_INVALID);
  CHECK(gdn_decode(pool, 0, ids, 4, x, ab, al, dt, cw + 1, y, nullptr) == GDN_ERR_INVALID);
  ids[2] = 3;
  CHECK(gdn_decode(pool, 0, ids, 4, x, ab, al, dt, cw, y, nullptr) == GDN_ERR_SLOTS);
  ids[2] = 8;
  CHECK(gdn_decode(pool, 1, ids, 4, x, ab, al, dt, cw, y, nullptr) == GDN_ERR_SLOTS);
  ids[2] = 6;
  // prefill: the pool's workspace grows; the fixed-scratch form refuses too many tokens
  int32_t* cu = dev_alloc<int32_t>(keep, 3);
  cu[0] = 0; cu[1] = 700; cu[2] = 1500;
  uint16_t* xp = dev_alloc<uint16_t>(keep, (size_t)1500 * D);
  uint16_t* abp = dev_alloc<uint16_t>(keep, (size_t)1500 * 64);
  uint16_t* yp = dev_alloc<uint16_t>(keep, (size_t)1500 * 32 * 128);
  CHECK(gdn_prefill_varlen(pool, 0, ids, cu, 2, 1500, xp, abp, al, dt, cw, yp, nullptr) == GDN_OK);
  CHECK(gdn_prefill_varlen_noalloc(pool, 0, ids, cu, 2, 1500, xp, abp, al, dt, cw, yp, nullptr) ==
        GDN_ERR_INVALID);
  CHECK(std::strstr(gdn_last_error(), "scratch") != nullptr);
  cu[1] = 300; cu[2] = 900;
  CHECK(gdn_prefill_varlen_noalloc(pool, 0, ids, cu, 2, 900, xp, abp, al, dt, cw, yp, nullptr) ==
        GDN_OK);
  ids[1] = 3;
  CHECK(gdn_prefill_varlen(pool, 0, ids, cu, 2, 900, xp, abp, al, dt, cw, yp, nullptr) ==
        GDN_ERR_SLOTS);
  // a long one-prompt split-path call (128 groups on 256 CUs) pipelines over
  // the pool's second stream (made on the first such call, reused by the
  // next, released with the pool); two prompts (256 groups) run in one pass
  ids[1] = 4;
  gdn_fake::split = true;
  cu[1] = 9000; cu[2] = 9000;
  uint16_t* xl = dev_alloc<uint16_t>(keep, (size_t)9000 * D);
  uint16_t* abl = dev_alloc<uint16_t>(keep, (size_t)9000 * 64);
  uint16_t* yl = dev_alloc<uint16_t>(keep, (size_t)9000 * 32 * 128);
  for (int k = 0; k < 2; ++k)
    CHECK(gdn_prefill_varlen(pool, 0, ids, cu, 1, 9000, xl, abl, al, dt, cw, yl, nullptr) == GDN_OK);
  cu[1] = 4000;
  CHECK(gdn_prefill_varlen(pool, 0, ids, cu, 2, 9000, xl, abl, al, dt, cw, yl, nullptr) == GDN_OK);
  gdn_fake::split = false;
  uint32_t flags = 1;
  CHECK(gdn_pool_check(pool, nullptr, &flags) == GDN_OK && flags == 0);
  CHECK(gdn_pool_destroy(pool) == GDN_OK);
  return 0;
}

static int test_kv() {
  gdn_kv_desc d{1, 8, 16, 4, 16, 2, 256, 256, 0, 0};
  gdn_kv* kv = nullptr;
  CHECK(gdn_kv_create(&d, &kv) == GDN_OK);
  int32_t free_pages = 0;
  int64_t len = 0;
  int32_t slots[4] = {2, 5, 0, 7}, ntok[4] = {100, 1, 64, 65};
  CHECK(gdn_kv_step(kv, 4, slots, ntok, nullptr) == GDN_OK);
  CHECK(gdn_kv_free_pages(kv, &free_pages) == GDN_OK && free_pages == 16 - (2 + 1 + 1 + 2));
  CHECK(gdn_kv_length(kv, 2, &len) == GDN_OK && len == 100);
  for (int step = 0; step < 40; ++step) {  // decode steps: slot 5 grows to 41 tokens
    int32_t one[4] = {1, 1, 1, 1};
    CHECK(gdn_kv_step(kv, 2, slots + 1, one, nullptr) == GDN_OK);
  }
  CHECK(gdn_kv_length(kv, 5, &len) == GDN_OK && len == 41);
  CHECK(gdn_kv_length(kv, 0, &len) == GDN_OK && len == 104);
  int32_t dup[2] = {3, 3}, two[2] = {1, 1};
  CHECK(gdn_kv_step(kv, 2, dup, two, nullptr) == GDN_ERR_INVALID);
  int32_t big[1] = {3}, nbig[1] = {257};
  CHECK(gdn_kv_step(kv, 1, big, nbig, nullptr) == GDN_ERR_INVALID);   // > max_step_tokens
  nbig[0] = 256;
  CHECK(gdn_kv_step(kv, 1, big, nbig, nullptr) == GDN_OK);            // 4 pages: slot full
  int32_t one1[1] = {1};
  CHECK(gdn_kv_step(kv, 1, big, one1, nullptr) == GDN_ERR_INVALID);   // > max_pages_per_slot
  CHECK(gdn_kv_free_pages(kv, &free_pages) == GDN_OK);
  int32_t pages_used = 0;
  for (int s = 0; s < 8; ++s) {
    CHECK(gdn_kv_length(kv, s, &len) == GDN_OK);
    pages_used += (int32_t)((len + 63) / 64);
  }
  CHECK(pages_used + free_pages == 16);
  int32_t s6[1] = {6}, n6[1] = {(free_pages + 1) * 64};
  if (n6[0] <= 256) {
    CHECK(gdn_kv_step(kv, 1, s6, n6, nullptr) == GDN_ERR_OOM);        // out of pages: no change
    int32_t fp2 = 0;
    CHECK(gdn_kv_free_pages(kv, &fp2) == GDN_OK && fp2 == free_pages);
  }
  for (int s = 0; s < 8; ++s) CHECK(gdn_kv_release(kv, s) == GDN_OK);
  CHECK(gdn_kv_free_pages(kv, &free_pages) == GDN_OK && free_pages == 16);
  CHECK(gdn_kv_release(kv, 8) == GDN_ERR_INVALID);
  CHECK(gdn_kv_destroy(kv) == GDN_OK);
  return 0;
}

static int test_exec() {
  std::vector<std::vector<char>> keep;
  const int hidden = 512, vocab = 1024, Hk = 16, Hv = 32, D = 2 * Hk * 128 + Hv * 128;
  gdn_pool_desc pd{2, 4, Hk, Hv, 128, 128, 4, 0};
  gdn_pool* pool = nullptr;
  CHECK(gdn_pool_create(&pd, &pool) == GDN_OK);
  gdn_layer* layers[2];
  std::vector<gdn_qlinear*> qls;
  for (int l = 0; l < 2; ++l) {
    gdn_qlinear* in = make_qlinear(keep, hidden, {D, Hv * 128, Hv, Hv});
    gdn_qlinear* out = make_qlinear(keep, Hv * 128, {hidden});
    CHECK(in && out);
    qls.push_back(in);
    qls.push_back(out);
    gdn_layer_desc ld{pool, l, in, out, dev_alloc<float>(keep, Hv), dev_alloc<float>(keep, Hv),
                      dev_alloc<uint16_t>(keep, (size_t)D * 4), dev_alloc<uint16_t>(keep, 128),
                      1e-6f};
    CHECK(gdn_layer_create(&ld, &layers[l]) == GDN_OK);
  }
  const int Hq = 16, Hkv = 2;
  gdn_qlinear* qkv = make_qlinear(keep, hidden, {Hq * 512 + 2 * Hkv * 256});
  gdn_qlinear* o = make_qlinear(keep, Hq * 256, {hidden});
  gdn_qlinear* head = make_qlinear(keep, hidden, {vocab});
  CHECK(qkv && o && head);
  qls.push_back(qkv);
  qls.push_back(o);
  qls.push_back(head);
  gdn_kv_desc kd{1, 4, 6, 4, Hq, Hkv, 256, 256, 0, 0};
  gdn_kv* kv = nullptr;
  CHECK(gdn_kv_create(&kd, &kv) == GDN_OK);
  gdn_exec_attn_layer al{1, qkv, o, dev_alloc<uint16_t>(keep, 256), dev_alloc<uint16_t>(keep, 256)};
  const uint16_t* norms[3] = {dev_alloc<uint16_t>(keep, hidden), dev_alloc<uint16_t>(keep, hidden),
                              dev_alloc<uint16_t>(keep, hidden)};
  gdn_exec_desc ed{};
  ed.pool = pool;
  ed.num_layers = 2;
  ed.layers = layers;
  ed.input_norm_w = norms;
  ed.final_norm_w = dev_alloc<uint16_t>(keep, hidden);
  ed.rms_eps = 1e-6f;
  ed.embed = dev_alloc<uint16_t>(keep, (size_t)vocab * hidden);
  ed.head = head;
  ed.max_batch = 4;
  ed.max_prompt = 300;  // > 4 pages per slot: refused
  ed.device = 0;
  ed.num_attn_layers = 1;
  ed.attn_layers = &al;
  ed.kv = kv;
  ed.rope_theta = 1e7f;
  ed.rotary_dim = 64;
  gdn_exec* ex = nullptr;
  CHECK(gdn_exec_create(&ed, nullptr, &ex) == GDN_ERR_INVALID && !ex);
  ed.max_prompt = 256;
  CHECK(gdn_exec_create(&ed, nullptr, &ex) == GDN_OK && ex);
  std::vector<int32_t> p1(10, 7), p23(70 + 5, 9);
  uint32_t t = 0, tb[4] = {0, 0, 0, 0};
  CHECK(gdn_exec_prefill(ex, 1, p1.data(), 10, &t) == GDN_OK && t == 0);
  uint64_t ids23[2] = {2, 3};
  int32_t lens23[2] = {70, 5};
  CHECK(gdn_exec_prefill_batch(ex, 2, ids23, p23.data(), lens23, tb) == GDN_OK);
  uint64_t ids[3] = {1, 2, 3};
  uint32_t toks[3] = {1, 2, 3}, next[3];
  for (int step = 0; step < 5; ++step)
    CHECK(gdn_exec_decode_batch(ex, ids, toks, 3, next) == GDN_OK);
  CHECK(gdn_exec_submit_batch(ex, ids, toks, 3) == GDN_OK);
  CHECK(gdn_exec_submit_batch(ex, ids, toks, 3) == GDN_ERR_INVALID);  // not collected yet
  CHECK(gdn_exec_collect_batch(ex, next, 2) == GDN_ERR_INVALID);
  CHECK(gdn_exec_collect_batch(ex, next, 3) == GDN_OK);
  CHECK(gdn_exec_collect_batch(ex, next, 3) == GDN_ERR_INVALID);      // nothing submitted
  // chained steps: the last submitted step's B, at most two uncollected, oldest first
  CHECK(gdn_exec_submit_next(ex, 3) == GDN_OK);
  CHECK(gdn_exec_submit_next(ex, 2) == GDN_ERR_INVALID);
  CHECK(gdn_exec_submit_next(ex, 3) == GDN_OK);
  CHECK(gdn_exec_submit_next(ex, 3) == GDN_ERR_INVALID);
  CHECK(gdn_exec_submit_batch(ex, ids, toks, 3) == GDN_ERR_INVALID);
  CHECK(gdn_exec_collect_batch(ex, next, 2) == GDN_ERR_INVALID);
  CHECK(gdn_exec_collect_batch(ex, next, 3) == GDN_OK);
  CHECK(gdn_exec_submit_next(ex, 3) == GDN_OK);
  for (int k = 0; k < 2; ++k) CHECK(gdn_exec_collect_batch(ex, next, 3) == GDN_OK);
  CHECK(gdn_exec_collect_batch(ex, next, 3) == GDN_ERR_INVALID);
  uint64_t bad[2] = {1, 9};
  CHECK(gdn_exec_decode_batch(ex, bad, toks, 2, next) == GDN_ERR_INVALID);
  uint64_t twice[2] = {1, 1};
  CHECK(gdn_exec_decode_batch(ex, twice, toks, 2, next) == GDN_ERR_INVALID);
  uint32_t oov[1] = {(uint32_t)vocab};
  CHECK(gdn_exec_decode_batch(ex, ids, oov, 1, next) == GDN_ERR_INVALID);
  // a restart that cannot get its KV pages fails before anything changes
  int32_t free_pages = 0, slot1 = -1, in_use = 0, slot_after = -1;
  CHECK(gdn_kv_free_pages(kv, &free_pages) == GDN_OK && free_pages == 2);
  CHECK(gdn_exec_seq_slot(ex, 1, &slot1) == GDN_OK);
  std::vector<int32_t> longp(256, 5);
  CHECK(gdn_exec_prefill(ex, 1, longp.data(), 256, &t) == GDN_ERR_OOM);
  CHECK(gdn_exec_submit_next(ex, 3) == GDN_ERR_INVALID);  // a prefill ends the chain
  CHECK(gdn_exec_seq_slot(ex, 1, &slot_after) == GDN_OK && slot_after == slot1);
  int32_t fp2 = 0;
  CHECK(gdn_kv_free_pages(kv, &fp2) == GDN_OK && fp2 == free_pages);
  // a failure after admission retires every sequence of the call
  CHECK(gdn_slots_in_use(pool, &in_use) == GDN_OK && in_use == 3);
  gdn_fake::fail_embed = true;
  uint64_t ids14[2] = {1, 4};
  int32_t lens14[2] = {3, 4};
  std::vector<int32_t> p14(7, 2);
  CHECK(gdn_exec_prefill_batch(ex, 2, ids14, p14.data(), lens14, tb) == GDN_ERR_HIP);
  gdn_fake::fail_embed = false;
  CHECK(gdn_exec_seq_slot(ex, 1, &slot_after) == GDN_ERR_INVALID);
  CHECK(gdn_exec_seq_slot(ex, 4, &slot_after) == GDN_ERR_INVALID);
  CHECK(gdn_slots_in_use(pool, &in_use) == GDN_OK && in_use == 2);
  int64_t len = -1;
  CHECK(gdn_kv_length(kv, slot1, &len) == GDN_OK && len == 0);
  // release, re-admission, and destroy with sequences still held
  CHECK(gdn_exec_release(ex, 2) == GDN_OK);
  CHECK(gdn_exec_release(ex, 2) == GDN_ERR_INVALID);
  CHECK(gdn_exec_prefill(ex, 2, p1.data(), 10, &t) == GDN_OK);
  CHECK(gdn_exec_destroy(ex) == GDN_OK);
  CHECK(gdn_slots_in_use(pool, &in_use) == GDN_OK && in_use == 0);
  CHECK(gdn_kv_free_pages(kv, &free_pages) == GDN_OK && free_pages == 6);
  for (gdn_layer* l : layers) CHECK(gdn_layer_destroy(l) == GDN_OK);
  for (gdn_qlinear* q : qls) CHECK(gdn_qlinear_destroy(q) == GDN_OK);
  CHECK(gdn_kv_destroy(kv) == GDN_OK);
  CHECK(gdn_pool_destroy(pool) == GDN_OK);
  return 0;
}

// The executor's step graphs hold the pool's activation buffer: after
// gdn_pool_reserve grows it, the next step drops every graph and captures anew.
static int test_exec_graphs_follow_pool_buffer() {
  std::vector<std::vector<char>> keep;
  const int hidden = 512, vocab = 1024, Hk = 16, Hv = 32, D = 2 * Hk * 128 + Hv * 128;
  gdn_pool_desc pd{1, 4, Hk, Hv, 128, 128, 4, 0};
  gdn_pool* pool = nullptr;
  CHECK(gdn_pool_create(&pd, &pool) == GDN_OK);
  gdn_qlinear* in = make_qlinear(keep, hidden, {D, Hv * 128, Hv, Hv});
  gdn_qlinear* out = make_qlinear(keep, Hv * 128, {hidden});
  gdn_qlinear* head = make_qlinear(keep, hidden, {vocab});
  CHECK(in && out && head);
  gdn_layer_desc ld{pool, 0, in, out, dev_alloc<float>(keep, Hv), dev_alloc<float>(keep, Hv),
                    dev_alloc<uint16_t>(keep, (size_t)D * 4), dev_alloc<uint16_t>(keep, 128),
                    1e-6f};
  gdn_layer* layer = nullptr;
  CHECK(gdn_layer_create(&ld, &layer) == GDN_OK);
  const uint16_t* norms[1] = {dev_alloc<uint16_t>(keep, hidden)};
  gdn_exec_desc ed{};
  ed.pool = pool;
  ed.num_layers = 1;
  ed.layers = &layer;
  ed.input_norm_w = norms;
  ed.final_norm_w = dev_alloc<uint16_t>(keep, hidden);
  ed.rms_eps = 1e-6f;
  ed.embed = dev_alloc<uint16_t>(keep, (size_t)vocab * hidden);
  ed.head = head;
  ed.max_batch = 4;
  ed.max_prompt = 64;
  ed.device = 0;
  gdn_fake::capture = true;
  gdn_fake::graphs_live = gdn_fake::graphs_destroyed = gdn_fake::graphs_made = 0;
  gdn_exec* ex = nullptr;
  CHECK(gdn_exec_create(&ed, nullptr, &ex) == GDN_OK && ex);
  std::vector<int32_t> p(5, 3);
  uint32_t t = 0;
  uint64_t ids[2] = {1, 2};
  CHECK(gdn_exec_prefill(ex, 1, p.data(), 5, &t) == GDN_OK);
  CHECK(gdn_exec_prefill(ex, 2, p.data(), 5, &t) == GDN_OK);
  uint32_t toks[2] = {1, 2}, next[2];
  CHECK(gdn_exec_decode_batch(ex, ids, toks, 2, next) == GDN_OK);
  const int made = gdn_fake::graphs_made;
  CHECK(made > 0 && gdn_fake::graphs_destroyed == 0);
  CHECK(gdn_exec_decode_batch(ex, ids, toks, 2, next) == GDN_OK);
  CHECK(gdn_fake::graphs_made == made);                      // replayed, not captured again
  CHECK(gdn_pool_reserve(pool, 4096, nullptr) == GDN_OK);    // activation buffer reallocated
  CHECK(gdn_exec_decode_batch(ex, ids, toks, 2, next) == GDN_OK);
  CHECK(gdn_fake::graphs_destroyed == made);                 // every old graph dropped
  CHECK(gdn_fake::graphs_made == 2 * made);                  // and captured anew
  CHECK(gdn_pool_reserve(pool, 4096, nullptr) == GDN_OK);    // no growth: graphs kept
  CHECK(gdn_exec_decode_batch(ex, ids, toks, 2, next) == GDN_OK);
  CHECK(gdn_fake::graphs_made == 2 * made);
  CHECK(gdn_exec_destroy(ex) == GDN_OK);
  CHECK(gdn_fake::graphs_live == 0);
  gdn_fake::capture = false;
  CHECK(gdn_layer_destroy(layer) == GDN_OK);
  for (gdn_qlinear* q : {in, out, head}) CHECK(gdn_qlinear_destroy(q) == GDN_OK);
  CHECK(gdn_pool_destroy(pool) == GDN_OK);
  return 0;
}

int main() {
  if (test_pool() || test_kv() || test_exec() || test_exec_graphs_follow_pool_buffer()) return 1;
  std::printf("ALL OK (%d checks)\n", g_checks);
  return 0;
}
