// Test-side stand-in for the HIP runtime calls and the device launches that
// libgdn's host code (gdn_api.cpp, gdn_exec.cpp, gdn_kv.cpp) makes, so that
// the host code -- pool and slot allocator, KV page planner, executor slot
// maps, error and rollback paths -- runs on the CPU under AddressSanitizer
// and UndefinedBehaviorSanitizer. Device memory is host memory, copies are
// memcpy, streams and events complete at once, and launches compute nothing
// except the greedy pick, which writes token 0 (a valid id) so that the
// executor's loops can proceed. Workspace sizes follow the library's own
// formulas closely enough for the host code's checks; the numbers are not
// tested here.
#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdlib>
#include <functional>
#include <vector>
#include <cstring>

#include "gdn_common.h"

namespace gdn_fake {
bool fail_embed = false;  // set by the test: embedding launches fail
bool capture = false;     // set by the test: stream capture records the stand-in launches
bool split = false;       // set by the test: prefill calls take the split path (2-wave groups)
int graphs_live = 0, graphs_destroyed = 0, graphs_made = 0;
std::vector<std::function<void()>>* recording = nullptr;  // the capture in progress
}

extern "C" {

hipError_t hipMalloc(void** ptr, size_t size) {
  *ptr = std::calloc(1, size ? size : 1);
  return *ptr ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void* ptr) {
  std::free(ptr);
  return hipSuccess;
}
hipError_t hipHostMalloc(void** ptr, size_t size, unsigned int) { return hipMalloc(ptr, size); }
hipError_t hipHostGetDevicePointer(void** dev, void* host, unsigned int) {
  *dev = host;
  return hipSuccess;
}
hipError_t hipHostFree(void* ptr) { return hipFree(ptr); }
hipError_t hipMemset(void* dst, int value, size_t n) {
  std::memset(dst, value, n);
  return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int value, size_t n, hipStream_t) {
  return hipMemset(dst, value, n);
}
hipError_t hipMemcpy(void* dst, const void* src, size_t n, hipMemcpyKind) {
  std::memcpy(dst, src, n);
  return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t n, hipMemcpyKind kind, hipStream_t) {
  return hipMemcpy(dst, src, n, kind);
}
hipError_t hipSetDevice(int id) { return id == 0 ? hipSuccess : hipErrorInvalidDevice; }
hipError_t hipGetDevice(int* id) {
  *id = 0;
  return hipSuccess;
}
hipError_t hipDeviceGetAttribute(int* value, hipDeviceAttribute_t attr, int) {
  *value = attr == hipDeviceAttributeMultiprocessorCount ? 256 : 0;
  return hipSuccess;
}
hipError_t hipGetDeviceCount(int* count) {
  *count = 1;
  return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
hipError_t hipStreamCreateWithFlags(hipStream_t* stream, unsigned) {
  *stream = reinterpret_cast<hipStream_t>(new char[8]);
  return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t stream) {
  delete[] reinterpret_cast<char*>(stream);
  return hipSuccess;
}
// Stream capture: refused unless the test sets gdn_fake::capture. Then the
// stand-in launches made while capturing are recorded instead of run (only the
// greedy pick has an effect here: it writes the picks) and a graph launch
// replays them, so the executor's host-side graph bookkeeping (capture,
// replay, drop) runs as on the device, counted by graphs_*.
hipError_t hipStreamBeginCapture(hipStream_t, hipStreamCaptureMode) {
  if (!gdn_fake::capture) return hipErrorNotSupported;
  gdn_fake::recording = new std::vector<std::function<void()>>();
  return hipSuccess;
}
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* status) {
  *status = gdn_fake::recording ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
  return hipSuccess;
}
hipError_t hipStreamEndCapture(hipStream_t, hipGraph_t* graph) {
  *graph = reinterpret_cast<hipGraph_t>(gdn_fake::recording);
  gdn_fake::recording = nullptr;
  return *graph ? hipSuccess : hipErrorNotSupported;
}
hipError_t hipGraphInstantiate(hipGraphExec_t* exec, hipGraph_t graph, hipGraphNode_t*, char*,
                               size_t) {
  if (!gdn_fake::capture || !graph) return hipErrorNotSupported;
  *exec = reinterpret_cast<hipGraphExec_t>(new std::vector<std::function<void()>>(
      *reinterpret_cast<std::vector<std::function<void()>>*>(graph)));
  ++gdn_fake::graphs_live;
  ++gdn_fake::graphs_made;
  return hipSuccess;
}
hipError_t hipGraphDestroy(hipGraph_t graph) {
  delete reinterpret_cast<std::vector<std::function<void()>>*>(graph);
  return hipSuccess;
}
hipError_t hipGraphExecDestroy(hipGraphExec_t exec) {
  if (exec) {
    delete reinterpret_cast<std::vector<std::function<void()>>*>(exec);
    --gdn_fake::graphs_live;
    ++gdn_fake::graphs_destroyed;
  }
  return hipSuccess;
}
hipError_t hipGraphLaunch(hipGraphExec_t exec, hipStream_t) {
  if (!gdn_fake::capture || !exec) return hipErrorNotSupported;
  for (auto& fn : *reinterpret_cast<std::vector<std::function<void()>>*>(exec)) fn();
  return hipSuccess;
}
hipError_t hipDeviceSynchronize(void) { return hipSuccess; }
hipError_t hipGetLastError(void) { return hipSuccess; }
const char* hipGetErrorString(hipError_t) { return "host stand-in"; }
hipError_t hipEventCreateWithFlags(hipEvent_t* event, unsigned) {
  *event = reinterpret_cast<hipEvent_t>(new char[8]);
  return hipSuccess;
}
hipError_t hipEventDestroy(hipEvent_t event) {
  delete[] reinterpret_cast<char*>(event);
  return hipSuccess;
}
hipError_t hipEventRecord(hipEvent_t, hipStream_t) { return hipSuccess; }
hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
hipError_t hipStreamQuery(hipStream_t) { return hipSuccess; }

}  // extern "C"

namespace gdn {

hipError_t launch_qlinear_pack(const QLinearPackArgs&) { return hipSuccess; }
int qlinear_decode_slices(int K, int Npad) {
  if (K <= 512 || (K <= 2048 && Npad / 64 >= 128) || Npad >= 131072) return 1;
  return K / 512;
}
hipError_t launch_qlinear(const QLinearArgs& a) {
  if (a.defer) *a.defer = QPartial{};
  if (a.M <= 64 && a.Npad < 131072 && a.part) {
    const int ns = qlinear_decode_slices(a.K, a.Npad);
    if (ns > 1 && a.defer) *a.defer = QPartial{a.part, ns, a.Npad};
  }
  return hipSuccess;
}
hipError_t launch_decode(const DecodeArgs&) { return hipSuccess; }
hipError_t launch_recurrent(const RecurrentArgs&) { return hipSuccess; }
hipError_t launch_slots(const SlotArgs&) { return hipSuccess; }
hipError_t launch_validate(const int32_t*, int, int, uint32_t*, hipStream_t) { return hipSuccess; }
int prefill_chunk_waves(int, int, int, int) { return gdn_fake::split ? 2 : 8; }
int prefill_pipeline_segments(int waves, int total_tokens, int groups, int cus) {
  return waves == 2 && 2 * groups <= cus && total_tokens >= 8192
             ? std::min(8, total_tokens / 4096)
             : 1;
}
size_t prefill_workspace_bytes(int R, int Hk, int T, int nseq, int waves, bool y_scratch) {
  const size_t Hv = (size_t)Hk * R;
  size_t b = (size_t)T * (2 * (size_t)Hk * kDk * 2 + Hv * kDv * 2 + Hv * 6) + 5 * 256;
  if (waves < 8) b += (size_t)(T / 64 + nseq) * Hv * 17408 + (y_scratch ? (size_t)T * Hv * kDv * 2 : 0);
  return b;
}
size_t prefill_workspace_reserve_bytes(int R, int Hk, int T) {
  return prefill_workspace_bytes(R, Hk, T, 1, 2, true);
}
static unsigned char g_scratch[(size_t)16 << 20];
size_t noalloc_scratch_bytes() { return sizeof(g_scratch); }
hipError_t noalloc_scratch(void** out) {
  *out = g_scratch;
  return hipSuccess;
}
hipError_t launch_prefill(const PrefillArgs&) { return hipSuccess; }
size_t attn_workspace_bytes(int T, int Hq, int64_t chunks) {
  return (size_t)T * Hq * 256 * 2 + (size_t)chunks * 16 * 260 * 4 + 256;
}
int attn_chunk_blocks() { return 24; }
hipError_t launch_attn(const AttnArgs&) { return hipSuccess; }
hipError_t launch_kv_gather(const uint16_t*, const int32_t*, int, int64_t, uint16_t*, uint16_t*,
                            hipStream_t) {
  return hipSuccess;
}
hipError_t launch_embed(const uint16_t*, const int32_t*, int, int, int, uint16_t*, hipStream_t) {
  return gdn_fake::fail_embed ? hipErrorLaunchFailure : hipSuccess;
}
hipError_t launch_add_norm(uint16_t*, const uint16_t*, const QPartial*, int, int, const uint16_t*,
                           float, uint16_t*, hipStream_t, uint16_t*) {
  return hipSuccess;
}
hipError_t launch_gather_rows(const uint16_t*, const int32_t*, int, int, uint16_t*, hipStream_t) {
  return hipSuccess;
}
int argmax_chunks(int vocab) { return (vocab + 8191) / 8192; }
hipError_t launch_embed_norm(const uint16_t*, const int32_t*, int, int, int, const uint16_t*, float,
                             uint16_t*, uint16_t*, hipStream_t, uint16_t*) {
  return gdn_fake::fail_embed ? hipErrorLaunchFailure : hipSuccess;
}
hipError_t launch_argmax(const uint16_t*, int64_t, int n, int, float*, int*, int32_t* out,
                         int32_t* out_host, hipStream_t) {
  auto run = [=] {
    for (int i = 0; i < n; ++i) out[i] = 0;
    if (out_host)
      for (int i = 0; i < n; ++i) out_host[i] = 0;
  };
  if (gdn_fake::recording)
    gdn_fake::recording->push_back(run);
  else
    run();
  return hipSuccess;
}

}  // namespace gdn
