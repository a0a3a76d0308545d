// gdn_api.cpp -- C ABI of libgdn: pool lifetime, slot allocator, argument
// validation and kernel launches. See include/gdn.h for the contract.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdlib>
#include <cstdio>
#include <set>
#include <string>
#include <vector>

#include "gdn.h"
#include "gdn_common.h"

namespace {

thread_local std::string g_err;

gdn_status fail(gdn_status code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

}  // namespace

gdn_status gdn::set_error(gdn_status code, const char* msg) {
  g_err = msg;
  return code;
}

namespace {

gdn_status hip_fail(hipError_t e, const char* what) {
  return fail(GDN_ERR_HIP, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// Makes the pool's device current for the duration of a call.
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev_) != hipSuccess) prev_ = -1;
    if (prev_ != dev) ok_ = hipSetDevice(dev) == hipSuccess;
  }
  ~DeviceGuard() {
    if (ok_ && prev_ >= 0) {
      int cur = -1;
      if (hipGetDevice(&cur) == hipSuccess && cur != prev_) (void)hipSetDevice(prev_);
    }
  }
  bool ok() const { return ok_; }

 private:
  int prev_ = -1;
  bool ok_ = true;
};

}  // namespace

struct gdn_pool {
  gdn_pool_desc d{};
  int R = 0, D = 0;
  size_t state_elems = 0;  // per slot per layer, f32
  size_t conv_elems = 0;   // per slot per layer, bf16
  std::vector<float*> state;
  std::vector<uint16_t*> conv;
  float** d_state_ptrs = nullptr;
  uint16_t** d_conv_ptrs = nullptr;
  uint32_t* d_status = nullptr;
  void* workspace = nullptr;
  size_t workspace_bytes = 0;
  void* act = nullptr;  // gdn_layer_* activations: projection rows, gated rows
  size_t act_bytes = 0;
  uint64_t act_gen = 0;  // bumped whenever act is reallocated (captured graphs hold it)
  std::set<int32_t> free_slots;
  std::vector<uint8_t> in_use;
  int cus = 0;  // compute units of the pool's device
  // pipelined prefill: a second stream and its events, made on first use
  hipStream_t aux = nullptr;
  hipEvent_t pipe_ev[gdn::kPrefillPipeEvents] = {};
};

namespace {

void release(gdn_pool* p) {
  for (float* s : p->state)
    if (s) (void)hipFree(s);
  for (uint16_t* c : p->conv)
    if (c) (void)hipFree(c);
  if (p->d_state_ptrs) (void)hipFree(p->d_state_ptrs);
  if (p->d_conv_ptrs) (void)hipFree(p->d_conv_ptrs);
  if (p->d_status) (void)hipFree(p->d_status);
  if (p->workspace) (void)hipFree(p->workspace);
  if (p->act) (void)hipFree(p->act);
  for (hipEvent_t e : p->pipe_ev)
    if (e) (void)hipEventDestroy(e);
  if (p->aux) (void)hipStreamDestroy(p->aux);
  delete p;
}

gdn_status check_layer(const gdn_pool* p, int32_t layer, bool allow_all) {
  if (!p) return fail(GDN_ERR_INVALID, "pool is NULL");
  if (allow_all && layer == GDN_ALL_LAYERS) return GDN_OK;
  if (layer < 0 || layer >= p->d.num_layers)
    return fail(GDN_ERR_INVALID, "layer %d outside [0, %d)", layer, p->d.num_layers);
  return GDN_OK;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Debug check of a call's slot list (range and uniqueness) on the host before
// any launch: on when the library is built with GDN_DEBUG_SLOTS defined or the
// environment has GDN_DEBUG_SLOTS set to a value other than 0. It copies the
// list to the host and waits for `stream`, so it is for debugging, not for
// graph capture. Without it a repeated id races inside the kernels and an
// out-of-range id only latches GDN_FLAG_BAD_SLOT.
bool debug_slots_on() {
#ifdef GDN_DEBUG_SLOTS
  return true;
#else
  const char* e = getenv("GDN_DEBUG_SLOTS");
  return e && e[0] && !(e[0] == '0' && e[1] == 0);
#endif
}

gdn_status debug_check_slots(const gdn_pool* pool, const int32_t* slot_ids, int32_t n,
                                    void* stream, const char* who) {
  if (!debug_slots_on() || n <= 0) return GDN_OK;
  std::vector<int32_t> ids(n);
  hipError_t e = hipMemcpyAsync(ids.data(), slot_ids, sizeof(int32_t) * n,
                                hipMemcpyDeviceToHost, as_stream(stream));
  if (e == hipSuccess) e = hipStreamSynchronize(as_stream(stream));
  if (e != hipSuccess) return hip_fail(e, "slot list check");
  std::vector<uint8_t> seen(pool->d.num_slots, 0);
  for (int32_t i = 0; i < n; ++i) {
    const int32_t s = ids[i];
    if (s < 0 || s >= pool->d.num_slots)
      return fail(GDN_ERR_SLOTS, "%s: slot id %d at %d outside [0, %d)", who, s, i,
                  pool->d.num_slots);
    if (seen[s]) return fail(GDN_ERR_SLOTS, "%s: slot id %d appears twice", who, s);
    seen[s] = 1;
  }
  return GDN_OK;
}


}  // namespace

extern "C" {

const char* gdn_last_error(void) { return g_err.c_str(); }

const char* gdn_version(void) { return "gdn 0.1 gfx950"; }

gdn_status gdn_pool_describe(const gdn_pool* pool, gdn_pool_desc* desc) {
  if (!pool || !desc) return fail(GDN_ERR_INVALID, "gdn_pool_describe: NULL argument");
  *desc = pool->d;
  return GDN_OK;
}

gdn_status gdn_pool_create(const gdn_pool_desc* desc, gdn_pool** out) {
  if (!desc || !out) return fail(GDN_ERR_INVALID, "desc/out is NULL");
  *out = nullptr;
  const gdn_pool_desc& d = *desc;
  if (d.num_layers < 1 || d.num_slots < 1 || d.num_k_heads < 1 || d.num_v_heads < 1)
    return fail(GDN_ERR_INVALID, "num_layers/num_slots/heads must be >= 1");
  if (d.num_v_heads % d.num_k_heads != 0)
    return fail(GDN_ERR_INVALID, "num_v_heads (%d) not a multiple of num_k_heads (%d)",
                d.num_v_heads, d.num_k_heads);
  const int R = d.num_v_heads / d.num_k_heads;
  if (R != 1 && R != 2 && R != 4)
    return fail(GDN_ERR_UNSUPPORTED, "num_v_heads/num_k_heads = %d not in {1,2,4}", R);
  if (d.head_k_dim != gdn::kDk || d.head_v_dim != gdn::kDv)
    return fail(GDN_ERR_UNSUPPORTED, "head dims %dx%d unsupported (compiled for 128x128)",
                d.head_k_dim, d.head_v_dim);
  if (d.conv_kernel != gdn::kConvK)
    return fail(GDN_ERR_UNSUPPORTED, "conv_kernel %d unsupported (compiled for 4)", d.conv_kernel);
  int ndev = 0;
  hipError_t e = hipGetDeviceCount(&ndev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount");
  if (d.device < 0 || d.device >= ndev)
    return fail(GDN_ERR_INVALID, "device %d outside [0, %d)", d.device, ndev);
  DeviceGuard guard(d.device);
  if (!guard.ok()) return fail(GDN_ERR_HIP, "hipSetDevice(%d) failed", d.device);

  gdn_pool* p = new gdn_pool();
  p->d = d;
  p->R = R;
  if (hipDeviceGetAttribute(&p->cus, hipDeviceAttributeMultiprocessorCount, d.device) != hipSuccess) {
    (void)hipGetLastError();
    p->cus = 0;  // unknown: no pipelined prefill
  }
  p->D = 2 * d.num_k_heads * gdn::kDk + d.num_v_heads * gdn::kDv;
  p->state_elems = (size_t)d.num_v_heads * gdn::kTileElems;
  p->conv_elems = (size_t)(gdn::kConvK - 1) * p->D;
  p->state.assign(d.num_layers, nullptr);
  p->conv.assign(d.num_layers, nullptr);
  const size_t sbytes = p->state_elems * sizeof(float) * (size_t)d.num_slots;
  const size_t cbytes = p->conv_elems * sizeof(uint16_t) * (size_t)d.num_slots;
  for (int l = 0; l < d.num_layers; ++l) {
    if (hipMalloc(&p->state[l], sbytes) != hipSuccess ||
        hipMalloc(&p->conv[l], cbytes) != hipSuccess) {
      (void)hipGetLastError();
      release(p);
      return fail(GDN_ERR_OOM, "hipMalloc of layer %d (%zu + %zu bytes) failed", l, sbytes,
                  cbytes);
    }
    if ((e = hipMemset(p->state[l], 0, sbytes)) != hipSuccess ||
        (e = hipMemset(p->conv[l], 0, cbytes)) != hipSuccess) {
      release(p);
      return hip_fail(e, "hipMemset(pool)");
    }
  }
  if (hipMalloc(&p->d_state_ptrs, sizeof(float*) * d.num_layers) != hipSuccess ||
      hipMalloc(&p->d_conv_ptrs, sizeof(uint16_t*) * d.num_layers) != hipSuccess ||
      hipMalloc(&p->d_status, sizeof(uint32_t)) != hipSuccess) {
    (void)hipGetLastError();
    release(p);
    return fail(GDN_ERR_OOM, "hipMalloc of pool tables failed");
  }
  if ((e = hipMemcpy(p->d_state_ptrs, p->state.data(), sizeof(float*) * d.num_layers,
                     hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemcpy(p->d_conv_ptrs, p->conv.data(), sizeof(uint16_t*) * d.num_layers,
                     hipMemcpyHostToDevice)) != hipSuccess ||
      (e = hipMemset(p->d_status, 0, sizeof(uint32_t))) != hipSuccess ||
      (e = hipDeviceSynchronize()) != hipSuccess) {
    release(p);
    return hip_fail(e, "pool table upload");
  }
  for (int32_t s = 0; s < d.num_slots; ++s) p->free_slots.insert(s);
  p->in_use.assign(d.num_slots, 0);
  *out = p;
  return GDN_OK;
}

gdn_status gdn_pool_destroy(gdn_pool* pool) {
  if (!pool) return GDN_OK;
  DeviceGuard guard(pool->d.device);
  hipError_t e = hipDeviceSynchronize();
  release(pool);
  if (e != hipSuccess) return hip_fail(e, "hipDeviceSynchronize before pool release");
  return GDN_OK;
}

gdn_status gdn_pool_layer_state(gdn_pool* pool, int32_t layer, float** state,
                                uint16_t** conv_state) {
  gdn_status st = check_layer(pool, layer, false);
  if (st) return st;
  if (state) *state = pool->state[layer];
  if (conv_state) *conv_state = pool->conv[layer];
  return GDN_OK;
}

gdn_status gdn_pool_slot_bytes(const gdn_pool* pool, size_t* state_bytes, size_t* conv_bytes) {
  if (!pool) return fail(GDN_ERR_INVALID, "pool is NULL");
  if (state_bytes) *state_bytes = pool->state_elems * sizeof(float);
  if (conv_bytes) *conv_bytes = pool->conv_elems * sizeof(uint16_t);
  return GDN_OK;
}

gdn_status gdn_pool_check(gdn_pool* pool, void* stream, uint32_t* flags) {
  if (!pool || !flags) return fail(GDN_ERR_INVALID, "pool/flags is NULL");
  DeviceGuard guard(pool->d.device);
  hipError_t e = hipStreamSynchronize(as_stream(stream));
  if (e != hipSuccess) return hip_fail(e, "hipStreamSynchronize");
  uint32_t v = 0;
  if ((e = hipMemcpy(&v, pool->d_status, sizeof(v), hipMemcpyDeviceToHost)) != hipSuccess)
    return hip_fail(e, "read status");
  if ((e = hipMemset(pool->d_status, 0, sizeof(v))) != hipSuccess) return hip_fail(e, "clear status");
  if ((e = hipDeviceSynchronize()) != hipSuccess) return hip_fail(e, "clear status sync");
  *flags = v;
  return GDN_OK;
}

gdn_status gdn_slot_alloc(gdn_pool* pool, int32_t* slot) {
  if (!pool || !slot) return fail(GDN_ERR_INVALID, "pool/slot is NULL");
  if (pool->free_slots.empty())
    return fail(GDN_ERR_SLOTS, "no free slot (pool holds %d)", pool->d.num_slots);
  const int32_t s = *pool->free_slots.begin();
  pool->free_slots.erase(pool->free_slots.begin());
  pool->in_use[s] = 1;
  *slot = s;
  return GDN_OK;
}

gdn_status gdn_slot_free(gdn_pool* pool, int32_t slot) {
  if (!pool) return fail(GDN_ERR_INVALID, "pool is NULL");
  if (slot < 0 || slot >= pool->d.num_slots)
    return fail(GDN_ERR_SLOTS, "slot %d outside [0, %d)", slot, pool->d.num_slots);
  if (!pool->in_use[slot]) return fail(GDN_ERR_SLOTS, "slot %d is not allocated", slot);
  pool->in_use[slot] = 0;
  pool->free_slots.insert(slot);
  return GDN_OK;
}

gdn_status gdn_slots_in_use(const gdn_pool* pool, int32_t* count) {
  if (!pool || !count) return fail(GDN_ERR_INVALID, "pool/count is NULL");
  *count = pool->d.num_slots - (int32_t)pool->free_slots.size();
  return GDN_OK;
}

static gdn_status slot_move(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t n,
                            float* sbuf, uint16_t* cbuf, gdn::SlotOp op, void* stream,
                            const char* what) {
  gdn_status st = check_layer(pool, layer, op == gdn::SlotOp::kZero);
  if (st) return st;
  if (n < 0) return fail(GDN_ERR_INVALID, "%s: n = %d < 0", what, n);
  if (n == 0) return GDN_OK;
  if (!slot_ids) return fail(GDN_ERR_INVALID, "%s: slot_ids is NULL", what);
  if (n > 65535) return fail(GDN_ERR_INVALID, "%s: n = %d > 65535", what, n);
  DeviceGuard guard(pool->d.device);
  gdn::SlotArgs a{};
  a.op = op;
  a.layers.state = pool->d_state_ptrs;
  a.layers.conv = pool->d_conv_ptrs;
  a.layer0 = layer == GDN_ALL_LAYERS ? 0 : layer;
  a.nlayers = layer == GDN_ALL_LAYERS ? pool->d.num_layers : 1;
  a.n = n;
  a.num_slots = pool->d.num_slots;
  a.Hv = pool->d.num_v_heads;
  a.R = pool->R;
  a.conv_elems = (int)pool->conv_elems;
  a.slot_ids = slot_ids;
  a.state_buf = sbuf;
  a.conv_buf = cbuf;
  a.status = pool->d_status;
  a.stream = as_stream(stream);
  hipError_t e = gdn::launch_slots(a);
  if (e != hipSuccess) return hip_fail(e, what);
  return GDN_OK;
}

gdn_status gdn_slots_zero(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t n,
                          void* stream) {
  return slot_move(pool, layer, slot_ids, n, nullptr, nullptr, gdn::SlotOp::kZero, stream,
                   "gdn_slots_zero");
}

gdn_status gdn_slots_read(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t n,
                          float* state_out, uint16_t* conv_out, void* stream) {
  return slot_move(pool, layer, slot_ids, n, state_out, conv_out, gdn::SlotOp::kRead, stream,
                   "gdn_slots_read");
}

gdn_status gdn_slots_write(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t n,
                           const float* state_in, const uint16_t* conv_in, void* stream) {
  return slot_move(pool, layer, slot_ids, n, const_cast<float*>(state_in),
                   const_cast<uint16_t*>(conv_in), gdn::SlotOp::kWrite, stream,
                   "gdn_slots_write");
}

gdn_status gdn_slots_validate(gdn_pool* pool, const int32_t* slot_ids, int32_t n, void* stream) {
  if (!pool) return fail(GDN_ERR_INVALID, "pool is NULL");
  if (n < 0) return fail(GDN_ERR_INVALID, "n = %d < 0", n);
  if (n == 0) return GDN_OK;
  if (!slot_ids) return fail(GDN_ERR_INVALID, "slot_ids is NULL");
  DeviceGuard guard(pool->d.device);
  hipError_t e = gdn::launch_validate(slot_ids, n, pool->d.num_slots, pool->d_status,
                                      as_stream(stream));
  if (e != hipSuccess) return hip_fail(e, "gdn_slots_validate");
  return GDN_OK;
}

gdn_status gdn_recurrent(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t B,
                         int32_t T, const uint16_t* q, const uint16_t* k, const uint16_t* v,
                         const float* g, const uint16_t* beta, uint16_t* y, void* stream) {
  gdn_status st = check_layer(pool, layer, false);
  if (st) return st;
  if (B < 0 || T < 0) return fail(GDN_ERR_INVALID, "B = %d, T = %d must be >= 0", B, T);
  if (B == 0 || T == 0) return GDN_OK;
  if (B > 65535) return fail(GDN_ERR_INVALID, "B = %d > 65535", B);
  if (!slot_ids || !q || !k || !v || !g || !beta || !y)
    return fail(GDN_ERR_INVALID, "gdn_recurrent: NULL tensor pointer");
  DeviceGuard guard(pool->d.device);
  st = debug_check_slots(pool, slot_ids, B, stream, "gdn_recurrent");
  if (st) return st;
  gdn::RecurrentArgs a{};
  a.R = pool->R;
  a.Hk = pool->d.num_k_heads;
  a.B = B;
  a.T = T;
  a.num_slots = pool->d.num_slots;
  a.state = pool->state[layer];
  a.slot_ids = slot_ids;
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.y = y;
  a.status = pool->d_status;
  a.stream = as_stream(stream);
  hipError_t e = gdn::launch_recurrent(a);
  if (e != hipSuccess) return hip_fail(e, "gdn_recurrent launch");
  return GDN_OK;
}

// Token tiles of 64 run along the grid's y axis (at most 65535).
constexpr int32_t kMaxPrefillTokens = 65535 * 64;
// qlinear rows per call: 65535 tiles of 128 rows
constexpr int32_t kMaxQLinearRows = 65535 * 128;

// Grows a pool-held device buffer to at least `need` bytes. Growing waits
// for the stream, so work still reading the old buffer has finished.
static gdn_status ensure_buffer(void*& buf, size_t& bytes, size_t need, void* stream,
                                const char* what, uint64_t* gen = nullptr) {
  if (need <= bytes) return GDN_OK;
  if (gen) ++*gen;
  if (buf) {
    hipError_t e = hipStreamSynchronize(as_stream(stream));
    if (e != hipSuccess) return hip_fail(e, "workspace grow sync");
    (void)hipFree(buf);
    buf = nullptr;
    bytes = 0;
  }
  if (hipMalloc(&buf, need) != hipSuccess) {
    (void)hipGetLastError();
    buf = nullptr;
    return fail(GDN_ERR_OOM, "%s workspace of %zu bytes", what, need);
  }
  bytes = need;
  return GDN_OK;
}

static gdn_status ensure_workspace(gdn_pool* pool, size_t need, void* stream, const char* what) {
  return ensure_buffer(pool->workspace, pool->workspace_bytes, need, stream, what);
}

// The pool's second stream and events for a pipelined prefill (default
// priority, not blocking on the null stream), made once on the pool's device.
// false when they cannot be made: the call then runs in one pass.
static bool ensure_pipeline(gdn_pool* pool) {
  if (pool->aux) return true;
  hipStream_t s = nullptr;
  if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  for (hipEvent_t& e : pool->pipe_ev) {
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      for (hipEvent_t& f : pool->pipe_ev)
        if (f) (void)hipEventDestroy(f), f = nullptr;
      (void)hipStreamDestroy(s);
      return false;
    }
  }
  pool->aux = s;
  return true;
}

// Shared checks and launch of the fused decode (gdn_decode, gdn_decode_gated).
static gdn_status decode_common(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t B,
                                const uint16_t* qkv, int64_t xstride, const uint16_t* ab,
                                int64_t ab_stride, const float* A_log, const float* dt_bias,
                                const uint16_t* conv_w, uint16_t* y, const uint16_t* norm_w,
                                float norm_eps, uint16_t* out, void* stream, const char* who) {
  gdn_status st = check_layer(pool, layer, false);
  if (st) return st;
  if (B < 0) return fail(GDN_ERR_INVALID, "%s: B = %d < 0", who, B);
  if (B == 0) return GDN_OK;
  if (B > 65535) return fail(GDN_ERR_INVALID, "%s: B = %d > 65535", who, B);
  if (B > pool->d.num_slots)
    return fail(GDN_ERR_INVALID, "%s: B = %d > num_slots = %d (slot ids must be distinct)", who, B,
                pool->d.num_slots);
  if (!slot_ids || !qkv || !ab || !A_log || !dt_bias || !conv_w)
    return fail(GDN_ERR_INVALID, "%s: NULL tensor pointer", who);
  if (reinterpret_cast<uintptr_t>(conv_w) % 8 != 0)
    return fail(GDN_ERR_INVALID, "%s: conv_w must be 8-byte aligned", who);
  DeviceGuard guard(pool->d.device);
  st = debug_check_slots(pool, slot_ids, B, stream, who);
  if (st) return st;
  gdn::DecodeArgs a{};
  a.R = pool->R;
  a.Hk = pool->d.num_k_heads;
  a.B = B;
  a.num_slots = pool->d.num_slots;
  a.state = pool->state[layer];
  a.conv = pool->conv[layer];
  a.slot_ids = slot_ids;
  a.mixed = qkv;
  a.xstride = xstride;
  a.ab = ab;
  a.ab_stride = ab_stride;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.conv_w = conv_w;
  a.y = y;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.out = out;
  a.status = pool->d_status;
  a.stream = as_stream(stream);
  hipError_t e = gdn::launch_decode(a);
  if (e != hipSuccess) return hip_fail(e, who);
  return GDN_OK;
}

gdn_status gdn_decode(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t B,
                      const uint16_t* mixed_qkv, const uint16_t* ab, const float* A_log,
                      const float* dt_bias, const uint16_t* conv_w, uint16_t* y, void* stream) {
  if (!y && B > 0) return fail(GDN_ERR_INVALID, "gdn_decode: NULL tensor pointer");
  return decode_common(pool, layer, slot_ids, B, mixed_qkv, pool ? pool->D : 0, ab,
                       pool ? 2 * pool->d.num_v_heads : 0, A_log, dt_bias, conv_w, y, nullptr,
                       0.0f, nullptr, stream, "gdn_decode");
}

gdn_status gdn_decode_gated(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t B,
                            const uint16_t* qkvz, int64_t row_stride, const uint16_t* ab,
                            int64_t ab_stride, const float* A_log, const float* dt_bias,
                            const uint16_t* conv_w, const uint16_t* norm_w, float norm_eps,
                            uint16_t* out, uint16_t* y, void* stream) {
  if (pool) {
    const int64_t need = (int64_t)pool->D + (int64_t)pool->d.num_v_heads * pool->d.head_v_dim;
    if (row_stride < need)
      return fail(GDN_ERR_INVALID, "gdn_decode_gated: row_stride %lld < D + Hv*Dv = %lld",
                  (long long)row_stride, (long long)need);
    if (ab_stride < 2 * pool->d.num_v_heads)
      return fail(GDN_ERR_INVALID, "gdn_decode_gated: ab_stride %lld < 2*Hv = %d",
                  (long long)ab_stride, 2 * pool->d.num_v_heads);
  }
  if (B > 0 && (!norm_w || !out))
    return fail(GDN_ERR_INVALID, "gdn_decode_gated: NULL norm_w / out");
  if (!(norm_eps >= 0.0f))
    return fail(GDN_ERR_INVALID, "gdn_decode_gated: norm_eps must be >= 0");
  return decode_common(pool, layer, slot_ids, B, qkvz, row_stride, ab, ab_stride, A_log, dt_bias,
                       conv_w, y, norm_w, norm_eps, out, stream, "gdn_decode_gated");
}

// Shared checks and launches of the varlen prefill (gdn_prefill_varlen,
// gdn_prefill_varlen_gated).
static gdn_status prefill_common(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                                 const int32_t* cu_seqlens, int32_t nseq, int32_t total_tokens,
                                 const uint16_t* qkv, int64_t xstride, const uint16_t* ab,
                                 int64_t ab_stride, const float* A_log, const float* dt_bias,
                                 const uint16_t* conv_w, uint16_t* y, const uint16_t* norm_w,
                                 float norm_eps, uint16_t* out, void* stream, const char* who,
                                 bool noalloc = false) {
  gdn_status st = check_layer(pool, layer, false);
  if (st) return st;
  if (nseq < 0 || total_tokens < 0)
    return fail(GDN_ERR_INVALID, "%s: nseq = %d, total_tokens = %d must be >= 0", who, nseq,
                total_tokens);
  if (nseq == 0) return GDN_OK;
  if (nseq > 65535) return fail(GDN_ERR_INVALID, "%s: nseq = %d > 65535", who, nseq);
  if (total_tokens > kMaxPrefillTokens)
    return fail(GDN_ERR_INVALID, "%s: total_tokens = %d > %d per call", who, total_tokens,
                kMaxPrefillTokens);
  if (!slot_ids || !cu_seqlens || !A_log || !dt_bias || !conv_w)
    return fail(GDN_ERR_INVALID, "%s: NULL pointer", who);
  if (total_tokens > 0 && (!qkv || !ab || (!y && !out)))
    return fail(GDN_ERR_INVALID, "%s: NULL token tensor", who);
  if (reinterpret_cast<uintptr_t>(conv_w) % 8 != 0)
    return fail(GDN_ERR_INVALID, "%s: conv_w must be 8-byte aligned", who);
  if (reinterpret_cast<uintptr_t>(qkv) % 16 != 0 || xstride % 8 != 0)
    return fail(GDN_ERR_INVALID, "%s: token rows must be 16-byte aligned (pointer %% 16 == 0, "
                "row stride %% 8 == 0)", who);
  DeviceGuard guard(pool->d.device);
  st = debug_check_slots(pool, slot_ids, nseq, stream, who);
  if (st) return st;
  // The no-allocation entry takes the library's schedule when its workspace
  // fits the fixed scratch, and otherwise the fused schedule, whose workspace
  // is the smallest.
  int waves = gdn::prefill_chunk_waves(pool->R, pool->d.num_k_heads, nseq, total_tokens);
  size_t need = gdn::prefill_workspace_bytes(pool->R, pool->d.num_k_heads, total_tokens, nseq,
                                             waves, out && !y);
  if (noalloc && waves != 8 && need > gdn::noalloc_scratch_bytes()) {
    waves = 8;
    need = gdn::prefill_workspace_bytes(pool->R, pool->d.num_k_heads, total_tokens, nseq, waves,
                                        out && !y);
  }
  void* ws = nullptr;
  size_t ws_bytes = 0;
  if (noalloc) {
    ws_bytes = gdn::noalloc_scratch_bytes();
    if (need > ws_bytes)
      return fail(GDN_ERR_INVALID,
                  "%s: %d tokens need %zu bytes of workspace; its fixed scratch holds %zu "
                  "(%zu bytes per token at these head counts)",
                  who, total_tokens, need, ws_bytes,
                  gdn::prefill_workspace_bytes(pool->R, pool->d.num_k_heads, 1, 1, 8, false));
    hipError_t e = gdn::noalloc_scratch(&ws);
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)");
  } else {
    st = ensure_workspace(pool, need, stream, "prefill");
    if (st) return st;
    ws = pool->workspace;
    ws_bytes = pool->workspace_bytes;
  }
  gdn::PrefillArgs a{};
  a.R = pool->R;
  a.Hk = pool->d.num_k_heads;
  a.nseq = nseq;
  a.total_tokens = total_tokens;
  a.num_slots = pool->d.num_slots;
  a.state = pool->state[layer];
  a.conv = pool->conv[layer];
  a.slot_ids = slot_ids;
  a.cu_seqlens = cu_seqlens;
  a.mixed = qkv;
  a.xstride = xstride;
  a.ab = ab;
  a.ab_stride = ab_stride;
  a.A_log = A_log;
  a.dt_bias = dt_bias;
  a.conv_w = conv_w;
  a.y = y;
  a.norm_w = norm_w;
  a.norm_eps = norm_eps;
  a.out = out;
  a.status = pool->d_status;
  a.waves = waves;
  a.workspace = ws;
  a.workspace_bytes = ws_bytes;
  a.stream = as_stream(stream);
  // The split path pipelines its segments over a second stream, except under
  // stream capture and in the no-allocation entry (which makes no objects).
  const int groups = pool->d.num_v_heads * nseq * (waves ? 8 / waves : 1);
  const int segs = gdn::prefill_pipeline_segments(waves, total_tokens, groups, pool->cus);
  if (!noalloc && segs > 1) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(a.stream, &cs) != hipSuccess) {
      (void)hipGetLastError();
      cs = hipStreamCaptureStatusActive;
    }
    if (cs == hipStreamCaptureStatusNone && ensure_pipeline(pool)) {
      a.aux = pool->aux;
      a.events = pool->pipe_ev;
      a.segments = segs;
    }
  }
  hipError_t e = gdn::launch_prefill(a);
  if (e != hipSuccess) return hip_fail(e, who);
  return GDN_OK;
}

gdn_status gdn_prefill_varlen(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                              const int32_t* cu_seqlens, int32_t nseq, int32_t total_tokens,
                              const uint16_t* mixed_qkv, const uint16_t* ab, const float* A_log,
                              const float* dt_bias, const uint16_t* conv_w, uint16_t* y,
                              void* stream) {
  if (!y && total_tokens > 0 && nseq > 0)
    return fail(GDN_ERR_INVALID, "gdn_prefill_varlen: NULL token tensor");
  return prefill_common(pool, layer, slot_ids, cu_seqlens, nseq, total_tokens, mixed_qkv,
                        pool ? pool->D : 0, ab, pool ? 2 * pool->d.num_v_heads : 0, A_log, dt_bias,
                        conv_w, y, nullptr, 0.0f, nullptr, stream, "gdn_prefill_varlen");
}

gdn_status gdn_prefill_varlen_noalloc(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                                      const int32_t* cu_seqlens, int32_t nseq,
                                      int32_t total_tokens, const uint16_t* mixed_qkv,
                                      const uint16_t* ab, const float* A_log, const float* dt_bias,
                                      const uint16_t* conv_w, uint16_t* y, void* stream) {
  if (!y && total_tokens > 0 && nseq > 0)
    return fail(GDN_ERR_INVALID, "gdn_prefill_varlen_noalloc: NULL token tensor");
  return prefill_common(pool, layer, slot_ids, cu_seqlens, nseq, total_tokens, mixed_qkv,
                        pool ? pool->D : 0, ab, pool ? 2 * pool->d.num_v_heads : 0, A_log, dt_bias,
                        conv_w, y, nullptr, 0.0f, nullptr, stream, "gdn_prefill_varlen_noalloc",
                        true);
}

gdn_status gdn_prefill_varlen_gated(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                                    const int32_t* cu_seqlens, int32_t nseq, int32_t total_tokens,
                                    const uint16_t* qkvz, int64_t row_stride, const uint16_t* ab,
                                    int64_t ab_stride, const float* A_log, const float* dt_bias,
                                    const uint16_t* conv_w, const uint16_t* norm_w,
                                    float norm_eps, uint16_t* out, uint16_t* y, void* stream) {
  if (pool) {
    const int64_t need = (int64_t)pool->D + (int64_t)pool->d.num_v_heads * pool->d.head_v_dim;
    if (row_stride < need)
      return fail(GDN_ERR_INVALID, "gdn_prefill_varlen_gated: row_stride %lld < D + Hv*Dv = %lld",
                  (long long)row_stride, (long long)need);
    if (ab_stride < 2 * pool->d.num_v_heads)
      return fail(GDN_ERR_INVALID, "gdn_prefill_varlen_gated: ab_stride %lld < 2*Hv = %d",
                  (long long)ab_stride, 2 * pool->d.num_v_heads);
  }
  if (nseq > 0 && total_tokens > 0 && (!norm_w || !out))
    return fail(GDN_ERR_INVALID, "gdn_prefill_varlen_gated: NULL norm_w / out");
  if (!(norm_eps >= 0.0f))
    return fail(GDN_ERR_INVALID, "gdn_prefill_varlen_gated: norm_eps must be >= 0");
  return prefill_common(pool, layer, slot_ids, cu_seqlens, nseq, total_tokens, qkvz, row_stride,
                        ab, ab_stride, A_log, dt_bias, conv_w, y, norm_w, norm_eps,
                        out, stream, "gdn_prefill_varlen_gated");
}


// ------------------------------------------------------------ qlinear --

struct gdn_qlinear {
  int K = 0, N = 0, Npad = 0, G = 0, device = 0;
  void* wp = nullptr;        // packed weights [Npad/16][K/128][64][4] u32
  uint16_t* sp = nullptr;    // packed scales  [Npad/16][K/128][16][2] bf16
  uint16_t* bias = nullptr;  // [Npad, G] bf16
  uint16_t* nsc = nullptr;   // [Npad, G] bf16, -128 * scales
  float* part = nullptr;     // K-slice partials of decode-sized calls [slices][64][Npad] f32
};

static void qlinear_release(gdn_qlinear* q) {
  if (!q) return;
  if (q->wp) (void)hipFree(q->wp);
  if (q->sp) (void)hipFree(q->sp);
  if (q->bias) (void)hipFree(q->bias);
  if (q->nsc) (void)hipFree(q->nsc);
  if (q->part) (void)hipFree(q->part);
  delete q;
}

gdn_status gdn_qlinear_create(int32_t K, int32_t nparts, const int32_t* part_rows,
                              const uint32_t* const* w, const uint16_t* const* scales,
                              const uint16_t* const* biases, int32_t group_size, int32_t bits,
                              int32_t device, void* stream, gdn_qlinear** out) {
  if (!out) return fail(GDN_ERR_INVALID, "gdn_qlinear_create: out is NULL");
  *out = nullptr;
  if (bits != 4 || group_size != 64)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_qlinear_create: bits = %d, group_size = %d (need 4, 64)",
                bits, group_size);
  if (K <= 0 || K % 512 != 0 || K > 4096)
    return fail(GDN_ERR_UNSUPPORTED, "gdn_qlinear_create: K = %d must be a multiple of 512 in "
                "[512, 4096]", K);
  if (nparts < 1 || nparts > 64 || !part_rows || !w || !scales || !biases)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_create: nparts = %d / NULL part arrays", nparts);
  int64_t N = 0;
  for (int i = 0; i < nparts; ++i) {
    if (part_rows[i] <= 0 || part_rows[i] % 16 != 0)
      return fail(GDN_ERR_UNSUPPORTED, "gdn_qlinear_create: part %d has %d rows (need a positive "
                  "multiple of 16)", i, part_rows[i]);
    if (!w[i] || !scales[i] || !biases[i])
      return fail(GDN_ERR_INVALID, "gdn_qlinear_create: part %d has a NULL tensor", i);
    N += part_rows[i];
  }
  if (N > (1 << 24)) return fail(GDN_ERR_INVALID, "gdn_qlinear_create: %lld rows", (long long)N);
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_create: device %d not present", device);
  DeviceGuard guard(device);
  if (!guard.ok()) return fail(GDN_ERR_HIP, "gdn_qlinear_create: hipSetDevice(%d) failed", device);

  gdn_qlinear* q = new gdn_qlinear();
  q->K = K;
  q->N = (int)N;
  q->Npad = (int)((N + 127) / 128 * 128);
  q->G = K / 64;
  q->device = device;
  const size_t wbytes = (size_t)q->Npad * K / 2, gbytes = (size_t)q->Npad * q->G * 2;
  const int slices = gdn::qlinear_decode_slices(K, q->Npad);
  const size_t pbytes = slices > 1 ? (size_t)slices * 64 * q->Npad * sizeof(float) : 0;
  if (hipMalloc(&q->wp, wbytes) != hipSuccess || hipMalloc(&q->sp, gbytes) != hipSuccess ||
      hipMalloc(&q->bias, gbytes) != hipSuccess || hipMalloc(&q->nsc, gbytes) != hipSuccess ||
      (pbytes && hipMalloc(&q->part, pbytes) != hipSuccess)) {
    qlinear_release(q);
    return fail(GDN_ERR_OOM, "gdn_qlinear_create: hipMalloc of %zu bytes failed",
                wbytes + 3 * gbytes);
  }
  hipStream_t s = as_stream(stream);
  hipError_t e;
  if ((e = hipMemsetAsync(q->wp, 0, wbytes, s)) != hipSuccess ||
      (e = hipMemsetAsync(q->sp, 0, gbytes, s)) != hipSuccess ||
      (e = hipMemsetAsync(q->bias, 0, gbytes, s)) != hipSuccess ||
      (e = hipMemsetAsync(q->nsc, 0, gbytes, s)) != hipSuccess) {
    qlinear_release(q);
    return hip_fail(e, "gdn_qlinear_create: clear");
  }
  int frag = 0;
  for (int i = 0; i < nparts; ++i) {
    gdn::QLinearPackArgs a{};
    a.w = w[i];
    a.s = scales[i];
    a.b = biases[i];
    a.N = part_rows[i];
    a.K = K;
    a.frag0 = frag;
    a.wp = q->wp;
    a.sp = q->sp;
    a.bias = q->bias;
    a.nsc = q->nsc;
    a.stream = s;
    if ((e = gdn::launch_qlinear_pack(a)) != hipSuccess) {
      qlinear_release(q);
      return hip_fail(e, "gdn_qlinear_create: pack");
    }
    frag += part_rows[i] / 16;
  }
  if ((e = hipStreamSynchronize(s)) != hipSuccess) {
    qlinear_release(q);
    return hip_fail(e, "gdn_qlinear_create: synchronize");
  }
  *out = q;
  return GDN_OK;
}

gdn_status gdn_qlinear_destroy(gdn_qlinear* q) {
  if (!q) return GDN_OK;
  DeviceGuard guard(q->device);
  qlinear_release(q);
  return GDN_OK;
}

gdn_status gdn_qlinear_dims(const gdn_qlinear* q, int32_t* K, int32_t* N) {
  if (!q) return fail(GDN_ERR_INVALID, "gdn_qlinear_dims: NULL layer");
  if (K) *K = q->K;
  if (N) *N = q->N;
  return GDN_OK;
}

gdn_status gdn_qlinear_forward(const gdn_qlinear* q, const uint16_t* x, int64_t x_stride,
                               int32_t M, uint16_t* y, int64_t y_stride, void* stream) {
  return gdn::qlinear_forward(q, x, x_stride, M, y, y_stride, stream, nullptr);
}

gdn_status gdn_qlinear_forward_sums(const gdn_qlinear* q, const uint16_t* x, int64_t x_stride,
                                    const uint16_t* group_sums, int32_t M, uint16_t* y,
                                    int64_t y_stride, void* stream) {
  if (M > 0 && !group_sums)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_forward_sums: NULL group_sums");
  if (reinterpret_cast<uintptr_t>(group_sums) % 2 != 0)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_forward_sums: group_sums must be 2-byte aligned");
  return gdn::qlinear_forward(q, x, x_stride, M, y, y_stride, stream, nullptr, group_sums);
}

gdn_status gdn_add_rms_norm(uint16_t* h, const uint16_t* d, int32_t n, int32_t hidden,
                            const uint16_t* w, float eps, uint16_t* hn, uint16_t* group_sums,
                            void* stream) {
  if (n < 0) return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: n = %d < 0", n);
  if (n == 0) return GDN_OK;
  if (n > 65535) return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: n = %d > 65535", n);
  if (!h || !w || !hn) return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: NULL tensor pointer");
  if (hidden < 8 || hidden > 4096 || hidden % 8 != 0)
    return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: hidden = %d not a multiple of 8 in [8, 4096]",
                hidden);
  for (const void* p : {(const void*)h, (const void*)d, (const void*)w, (const void*)hn})
    if (reinterpret_cast<uintptr_t>(p) % 16 != 0)
      return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: h, d, w and hn need 16-byte alignment");
  if (!(eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: eps must be >= 0");
  if (group_sums && (n > 64 || hidden % 64 != 0))
    return fail(GDN_ERR_INVALID, "gdn_add_rms_norm: group_sums need n <= 64 (got %d) and hidden "
                "a multiple of 64 (got %d)", n, hidden);
  hipError_t e = gdn::launch_add_norm(h, d, nullptr, n, hidden, w, eps, hn, as_stream(stream),
                                      group_sums);
  if (e != hipSuccess) return hip_fail(e, "gdn_add_rms_norm launch");
  return GDN_OK;
}

}  // extern "C"

namespace gdn {

uint64_t pool_act_generation(const gdn_pool* p) { return p ? p->act_gen : 0; }

gdn_status qlinear_forward(const gdn_qlinear* q, const uint16_t* x, int64_t x_stride, int32_t M,
                           uint16_t* y, int64_t y_stride, void* stream, QPartial* defer,
                           const uint16_t* xsplit) {
  if (defer) *defer = QPartial{};
  if (!q) return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: NULL layer");
  if (M < 0) return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: M = %d < 0", M);
  if (M == 0) return GDN_OK;
  if (M > kMaxQLinearRows)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: M = %d > %d", M, kMaxQLinearRows);
  if (!x || !y) return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: NULL tensor pointer");
  if (x_stride < q->K || x_stride % 8 != 0 || reinterpret_cast<uintptr_t>(x) % 16 != 0)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: x needs 16-byte alignment and a row "
                "stride >= K that is a multiple of 8 (got %lld)", (long long)x_stride);
  if (y_stride < q->N || y_stride % 4 != 0 || reinterpret_cast<uintptr_t>(y) % 8 != 0)
    return fail(GDN_ERR_INVALID, "gdn_qlinear_forward: y needs 8-byte alignment and a row "
                "stride >= N that is a multiple of 4 (got %lld)", (long long)y_stride);
  DeviceGuard guard(q->device);
  gdn::QLinearArgs a{};
  a.x = x;
  a.xs = x_stride;
  a.M = M;
  a.K = q->K;
  a.N = q->N;
  a.Npad = q->Npad;
  a.wp = q->wp;
  a.sp = q->sp;
  a.bias = q->bias;
  a.nsc = q->nsc;
  a.y = y;
  a.ys = y_stride;
  a.part = q->part;
  a.defer = defer;
  a.xsplit = M <= 64 ? xsplit : nullptr;
  a.stream = as_stream(stream);
  hipError_t e = gdn::launch_qlinear(a);
  if (e != hipSuccess) return hip_fail(e, "gdn_qlinear_forward launch");
  return GDN_OK;
}

}  // namespace gdn

// ------------------------------------------------------------ gdn_layer --
// One GatedDeltaNet layer end to end (GatedDeltaNet::forward_with_cache,
// qwen3_5.rs:558-668): merged input projection -> conv / norm / gates /
// recurrence / RMSNormGated -> out_proj. Three launches per call (four with
// prefill's conv-state and chunk kernels); activations live in the pool's
// activation buffer.
struct gdn_layer {
  gdn_pool* pool = nullptr;
  int32_t layer = 0;
  const gdn_qlinear* in_proj = nullptr;
  const gdn_qlinear* out_proj = nullptr;
  const float* A_log = nullptr;
  const float* dt_bias = nullptr;
  const uint16_t* conv_w = nullptr;
  const uint16_t* norm_w = nullptr;
  float norm_eps = 0.0f;
  int64_t proj_stride = 0;  // row stride of the projection rows (N rounded up to 8)
};

namespace {

// Bytes of activations for ntok tokens: projection rows [ntok, proj_stride]
// then gated rows [ntok, Hv*Dv], both bf16 (the second starts 16-byte aligned
// because proj_stride is a multiple of 8).
size_t layer_act_bytes(const gdn_pool* p, int64_t ntok) {
  const int64_t n = (int64_t)p->D + 2LL * p->d.num_v_heads * p->d.head_v_dim + 2 * p->d.num_v_heads;
  const int64_t stride = (n + 7) & ~7LL;
  return (size_t)ntok * (size_t)(stride + (int64_t)p->d.num_v_heads * p->d.head_v_dim) * 2;
}

gdn_status layer_args(const gdn_layer* L, const uint16_t* x, int64_t x_stride, uint16_t* out,
                      int64_t out_stride, const char* who) {
  if (!L) return fail(GDN_ERR_INVALID, "%s: NULL layer", who);
  if (!x || !out) return fail(GDN_ERR_INVALID, "%s: NULL x / out", who);
  const int hidden = L->in_proj->K;
  if (x_stride < hidden || out_stride < hidden)
    return fail(GDN_ERR_INVALID, "%s: row strides (%lld, %lld) below the hidden size %d", who,
                (long long)x_stride, (long long)out_stride, hidden);
  return GDN_OK;
}

}  // namespace

extern "C" {

gdn_status gdn_layer_create(const gdn_layer_desc* desc, gdn_layer** out) {
  if (!desc || !out) return fail(GDN_ERR_INVALID, "gdn_layer_create: desc/out is NULL");
  *out = nullptr;
  const gdn_layer_desc& d = *desc;
  gdn_status st = check_layer(d.pool, d.layer, false);
  if (st) return st;
  if (!d.in_proj || !d.out_proj || !d.A_log || !d.dt_bias || !d.conv_w || !d.norm_w)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: NULL weight");
  if (reinterpret_cast<uintptr_t>(d.conv_w) % 8 != 0)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: conv_w must be 8-byte aligned");
  if (!(d.norm_eps >= 0.0f)) return fail(GDN_ERR_INVALID, "gdn_layer_create: norm_eps < 0");
  const gdn_pool* p = d.pool;
  const int Hv = p->d.num_v_heads, value = Hv * p->d.head_v_dim;
  const int n_in = p->D + value + 2 * Hv;
  if (d.in_proj->N != n_in)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: in_proj has %d outputs, the layer needs "
                "D + Hv*Dv + 2*Hv = %d (q|k|v|z|b|a)", d.in_proj->N, n_in);
  if (d.out_proj->K != value)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: out_proj input width %d != Hv*Dv = %d",
                d.out_proj->K, value);
  if (d.out_proj->N != d.in_proj->K)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: out_proj width %d != in_proj input width %d",
                d.out_proj->N, d.in_proj->K);
  if (d.in_proj->device != p->d.device || d.out_proj->device != p->d.device)
    return fail(GDN_ERR_INVALID, "gdn_layer_create: projections and pool on different devices");
  gdn_layer* L = new gdn_layer;
  L->pool = d.pool;
  L->layer = d.layer;
  L->in_proj = d.in_proj;
  L->out_proj = d.out_proj;
  L->A_log = d.A_log;
  L->dt_bias = d.dt_bias;
  L->conv_w = d.conv_w;
  L->norm_w = d.norm_w;
  L->norm_eps = d.norm_eps;
  L->proj_stride = ((int64_t)n_in + 7) & ~7LL;
  *out = L;
  return GDN_OK;
}

gdn_status gdn_layer_destroy(gdn_layer* layer) {
  delete layer;
  return GDN_OK;
}

gdn_status gdn_pool_reserve(gdn_pool* pool, int32_t max_tokens, void* stream) {
  gdn_status st = check_layer(pool, 0, false);
  if (st) return st;
  if (max_tokens < 0 || max_tokens > kMaxPrefillTokens)
    return fail(GDN_ERR_INVALID, "gdn_pool_reserve: max_tokens = %d outside [0, %d]", max_tokens,
                kMaxPrefillTokens);
  DeviceGuard guard(pool->d.device);
  st = ensure_buffer(pool->act, pool->act_bytes, layer_act_bytes(pool, max_tokens), stream,
                     "layer activation", &pool->act_gen);
  if (st) return st;
  return ensure_workspace(pool, gdn::prefill_workspace_reserve_bytes(pool->R, pool->d.num_k_heads,
                                                                     max_tokens), stream, "prefill");
}

gdn_status gdn_layer_decode(gdn_layer* L, const int32_t* slot_ids, int32_t B, const uint16_t* x,
                            int64_t x_stride, uint16_t* out, int64_t out_stride, void* stream) {
  return gdn::layer_decode(L, slot_ids, B, x, x_stride, out, out_stride, stream, nullptr);
}

}  // extern "C"

gdn_status gdn::layer_decode(gdn_layer* L, const int32_t* slot_ids, int32_t B, const uint16_t* x,
                             int64_t x_stride, uint16_t* out, int64_t out_stride, void* stream,
                             QPartial* defer, const uint16_t* xsplit) {
  if (defer) *defer = QPartial{};
  if (B == 0 && L) return GDN_OK;
  gdn_status st = layer_args(L, x, x_stride, out, out_stride, "gdn_layer_decode");
  if (st) return st;
  gdn_pool* p = L->pool;
  if (B < 0 || B > p->d.num_slots)
    return fail(GDN_ERR_INVALID, "gdn_layer_decode: B = %d outside [0, num_slots = %d]", B,
                p->d.num_slots);
  {
    DeviceGuard guard(p->d.device);
    st = ensure_buffer(p->act, p->act_bytes, layer_act_bytes(p, B), stream, "layer activation",
                       &p->act_gen);
    if (st) return st;
  }
  const int64_t value = (int64_t)p->d.num_v_heads * p->d.head_v_dim;
  uint16_t* proj = static_cast<uint16_t*>(p->act);
  uint16_t* gated = proj + (size_t)B * L->proj_stride;
  st = qlinear_forward(L->in_proj, x, x_stride, B, proj, L->proj_stride, stream, nullptr, xsplit);
  if (st) return st;
  st = gdn_decode_gated(p, L->layer, slot_ids, B, proj, L->proj_stride, proj + p->D + value,
                        L->proj_stride, L->A_log, L->dt_bias, L->conv_w, L->norm_w, L->norm_eps,
                        gated, nullptr, stream);
  if (st) return st;
  return qlinear_forward(L->out_proj, gated, value, B, out, out_stride, stream, defer);
}

extern "C" {

gdn_status gdn_layer_prefill(gdn_layer* L, const int32_t* slot_ids, const int32_t* cu_seqlens,
                             int32_t nseq, int32_t total_tokens, const uint16_t* x,
                             int64_t x_stride, uint16_t* out, int64_t out_stride, void* stream) {
  if ((nseq == 0 || total_tokens == 0) && L && nseq >= 0 && total_tokens >= 0) {
    if (nseq == 0) return GDN_OK;
    // empty sequences only: no tokens to project, the slots keep their state
    return gdn_prefill_varlen_gated(L->pool, L->layer, slot_ids, cu_seqlens, nseq, 0, nullptr,
                                    L->proj_stride, nullptr, L->proj_stride, L->A_log, L->dt_bias,
                                    L->conv_w, L->norm_w, L->norm_eps, nullptr, nullptr, stream);
  }
  gdn_status st = layer_args(L, x, x_stride, out, out_stride, "gdn_layer_prefill");
  if (st) return st;
  gdn_pool* p = L->pool;
  if (total_tokens < 0 || total_tokens > kMaxPrefillTokens)
    return fail(GDN_ERR_INVALID, "gdn_layer_prefill: total_tokens = %d outside [0, %d]",
                total_tokens, kMaxPrefillTokens);
  {
    DeviceGuard guard(p->d.device);
    st = ensure_buffer(p->act, p->act_bytes, layer_act_bytes(p, total_tokens), stream,
                       "layer activation", &p->act_gen);
    if (st) return st;
  }
  const int64_t value = (int64_t)p->d.num_v_heads * p->d.head_v_dim;
  uint16_t* proj = static_cast<uint16_t*>(p->act);
  uint16_t* gated = proj + (size_t)total_tokens * L->proj_stride;
  st = gdn_qlinear_forward(L->in_proj, x, x_stride, total_tokens, proj, L->proj_stride, stream);
  if (st) return st;
  st = gdn_prefill_varlen_gated(p, L->layer, slot_ids, cu_seqlens, nseq, total_tokens, proj,
                                L->proj_stride, proj + p->D + value, L->proj_stride, L->A_log,
                                L->dt_bias, L->conv_w, L->norm_w, L->norm_eps, gated, nullptr,
                                stream);
  if (st) return st;
  return gdn_qlinear_forward(L->out_proj, gated, value, total_tokens, out, out_stride, stream);
}

}  // extern "C"
