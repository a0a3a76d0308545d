// gdn_prefill.hip -- varlen prefill of packed sequences (cu_seqlens).
//
// The reference runs prefill one sequence at a time (B=1) through
// GatedDeltaNet::forward_with_cache with S>1 (qwen3_5.rs:611-658): conv1d
// over [conv_state | x], silu, split, q/k rms-norm, gates, and one
// gated_delta_kernel launch with T=S (metal_gdn.rs:37). Here any number of
// sequences share the launches, each addressed by its slot:
//   1. conv_kernel       (token, channel) parallel conv + silu -> xc
//   2. conv_state_kernel last K-1 rows of [conv_state | x] -> slot
//   3. prep_kernel       q/k rms-norm -> qn/kn, gates -> beta, g
//   4. recurrence        sequential per (sequence, key head) over tokens
// Workspace layout (each region 256-byte aligned):
//   xc [T,D] bf16 | qn [T,Hk,Dk] bf16 | kn [T,Hk,Dk] bf16 | beta [T,Hv] bf16 | g [T,Hv] f32

#include "gdn_common.h"

namespace gdn {

namespace {

constexpr float kQNormW = 0.0078125f;
constexpr float kKNormW = 0.08837890625f;
constexpr float kNormEps = 1e-6f;

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Workspace {
  uint16_t* xc;
  uint16_t* qn;
  uint16_t* kn;
  uint16_t* beta;
  float* g;
};

size_t carve(void* base, int R, int Hk, int T, Workspace* w) {
  const int Hv = Hk * R;
  const size_t D = 2 * (size_t)Hk * kDk + (size_t)Hv * kDv;
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) {
    void* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  Workspace ws;
  ws.xc = static_cast<uint16_t*>(take((size_t)T * D * 2));
  ws.qn = static_cast<uint16_t*>(take((size_t)T * Hk * kDk * 2));
  ws.kn = static_cast<uint16_t*>(take((size_t)T * Hk * kDk * 2));
  ws.beta = static_cast<uint16_t*>(take((size_t)T * Hv * 2));
  ws.g = static_cast<float*>(take((size_t)T * Hv * 4));
  if (w) *w = ws;
  return off;
}

// Index of the sequence holding token t: largest s with cu[s] <= t.
__device__ __forceinline__ int seq_of(const int32_t* __restrict__ cu, int nseq, int t) {
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (cu[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

}  // namespace

// 1. conv1d + silu (qwen3_5.rs:617-623): out[t,ch] = silu(sum_k padded[t+k,ch] w[ch,k])
// with padded = [slot conv state (K-1 rows) | x of the sequence]; f32
// accumulation, one rounding to bf16. grid (T, D/256), block 256.
__global__ __launch_bounds__(256) void prefill_conv_kernel(
    const uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int nseq, int num_slots, int D,
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ conv_w,
    uint16_t* __restrict__ xc) {
  const int t = blockIdx.x;
  const int ch = blockIdx.y * 256 + threadIdx.x;
  if (ch >= D) return;
  const int s = seq_of(cu, nseq, t);
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) return;  // flagged by the recurrence kernel
  // seq_of gives cu[s] <= t for a well-formed cu_seqlens; the clamp keeps the
  // conv-state row index in [0, K-1) for any input.
  const int st = min(max(cu[s], 0), t);
  const uint16_t* cs = conv + (size_t)slot * (kConvK - 1) * D;
  const uint2 wv = *reinterpret_cast<const uint2*>(conv_w + (size_t)ch * kConvK);
  const uint16_t wk[4] = {(uint16_t)(wv.x & 0xffffu), (uint16_t)(wv.x >> 16),
                          (uint16_t)(wv.y & 0xffffu), (uint16_t)(wv.y >> 16)};
  float acc = 0.0f;
#pragma unroll
  for (int k = 0; k < kConvK; ++k) {
    const int u = t + k - (kConvK - 1);  // source token
    const uint16_t p = u >= st ? x[(size_t)u * D + ch] : cs[(size_t)(u - st + kConvK - 1) * D + ch];
    acc += bf2f(p) * bf2f(wk[k]);
  }
  xc[(size_t)t * D + ch] = f2bf(silu_bf16(rbf(acc)));
}

// 2. new conv state = last K-1 rows of padded (qwen3_5.rs:618-619).
// Runs after (1) has read the old rows. grid (nseq, D/256), block 256.
__global__ __launch_bounds__(256) void prefill_conv_state_kernel(
    uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int num_slots, int D, int T, const uint16_t* __restrict__ x) {
  const int s = blockIdx.x;
  const int ch = blockIdx.y * 256 + threadIdx.x;
  if (ch >= D) return;
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) return;
  // Clamped so a malformed cu_seqlens cannot address outside x or the slot.
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  const int len = en - st;
  uint16_t* cs = conv + (size_t)slot * (kConvK - 1) * D;
  // padded row p: p < K-1 -> old state row p, else token st + p - (K-1).
  // New row j = padded row len + j; reading rows > j before writing row j
  // keeps the in-place update exact.
#pragma unroll
  for (int j = 0; j < kConvK - 1; ++j) {
    const int p = len + j;
    const uint16_t v = p < kConvK - 1 ? cs[(size_t)p * D + ch]
                                      : x[(size_t)(st + p - (kConvK - 1)) * D + ch];
    cs[(size_t)j * D + ch] = v;
  }
}

// 3. q/k rms-norm with the baked weights and the gates, per (token, hk).
// grid (T, Hk), block 256: threads 0..127 q, 128..255 k.
template <int R>
__global__ __launch_bounds__(256) void prefill_prep_kernel(
    int Hk, int D, const uint16_t* __restrict__ xc, const uint16_t* __restrict__ ab,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    uint16_t* __restrict__ qn, uint16_t* __restrict__ kn, uint16_t* __restrict__ beta,
    float* __restrict__ g) {
  const int t = blockIdx.x, hk = blockIdx.y;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int Hv = Hk * R;
  __shared__ float red[4];
  const int isk = tid >> 7, d = tid & 127;
  const float xv = bf2f(xc[(size_t)t * D + (size_t)isk * Hk * kDk + hk * kDk + d]);
  const float ss = wave_sum(xv * xv);
  if (lane == 0) red[wave] = ss;
  __syncthreads();
  const float sum = isk ? red[2] + red[3] : red[0] + red[1];
  const float rn = 1.0f / sqrtf(sum / (float)kDk + kNormEps);
  const float w = isk ? kKNormW : kQNormW;
  uint16_t* dst = isk ? kn : qn;
  dst[((size_t)t * Hk + hk) * kDk + d] = f2bf(w * rbf(xv * rn));
  if (tid < R) {
    const int h = hk * R + tid;
    const float braw = bf2f(ab[(size_t)t * 2 * Hv + h]);
    const float araw = bf2f(ab[(size_t)t * 2 * Hv + Hv + h]);
    beta[(size_t)t * Hv + h] = f2bf(sigmoid_f32(braw));
    const float sp = logf(expf(araw + dt_bias[h]) + 1.0f);
    g[(size_t)t * Hv + h] = expf(-(expf(A_log[h]) * sp));
  }
}

// 4. Sequential recurrence per (sequence, hk) over the sequence's tokens,
// state in the slot (metal_gdn.rs:37-62). Thread layout as in the decode
// kernels: 256-thread tile teams, rows grp+32i, cols 4(sub+8j)+e.
// grid (Hk, nseq), block 256*R.
template <int R>
__global__ __launch_bounds__(256 * R) void prefill_seq_recurrence_kernel(
    float* __restrict__ state, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int num_slots, int Hk, int D, int T,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ xc, const float* __restrict__ g,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y, uint32_t* __restrict__ status) {
  constexpr int NT = 256 * R;
  const int hk = blockIdx.x, s = blockIdx.y;
  const int Hv = Hk * R;
  const int tid = threadIdx.x;
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  if (en <= st) return;
  __shared__ __align__(16) float qs[kDk];
  __shared__ __align__(16) float ks[kDk];
  __shared__ float vs[R * kDv];
  __shared__ float red[2];
  __shared__ float gg[R], bb[R];
  const int r = tid >> 8;
  const int lt = tid & 255, grp = lt >> 3, sub = lt & 7;
  const int hv = hk * R + r;
  const int wave = tid >> 6, lane = tid & 63;
  float* tile = state + ((size_t)slot * Hv + hv) * kTileElems;
  float4 sreg[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      sreg[i][j] = *reinterpret_cast<const float4*>(tile + (grp + 32 * i) * kDk + 4 * (sub + 8 * j));
  const size_t voff = 2 * (size_t)Hk * kDk + (size_t)hk * R * kDv;
  for (int t = st; t < en; ++t) {
    if (tid < kDk) {
      const float qv = bf2f(qn[((size_t)t * Hk + hk) * kDk + tid]);
      const float kv = bf2f(kn[((size_t)t * Hk + hk) * kDk + tid]);
      qs[tid] = qv;
      ks[tid] = kv;
      const float p = wave_sum(qv * kv);
      if (lane == 0) red[wave] = p;
    }
    for (int c = tid; c < R * kDv; c += NT) vs[c] = bf2f(xc[(size_t)t * D + voff + c]);
    if (tid < R) {
      gg[tid] = g[(size_t)t * Hv + hk * R + tid];
      bb[tid] = bf2f(beta[(size_t)t * Hv + hk * R + tid]);
    }
    __syncthreads();
    const float kq = red[0] + red[1];
    const float gt = gg[r], bt = bb[r];
    float4 kk[4], qq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kk[j] = *reinterpret_cast<const float4*>(&ks[4 * (sub + 8 * j)]);
      qq[j] = *reinterpret_cast<const float4*>(&qs[4 * (sub + 8 * j)]);
    }
    float kd[4], qd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = 0.f, c = 0.f;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float4 sv = sreg[i][j];
        sv.x *= gt; sv.y *= gt; sv.z *= gt; sv.w *= gt;
        a += sv.x * kk[j].x + sv.y * kk[j].y + sv.z * kk[j].z + sv.w * kk[j].w;
        c += sv.x * qq[j].x + sv.y * qq[j].y + sv.z * qq[j].z + sv.w * qq[j].w;
        sreg[i][j] = sv;
      }
      kd[i] = sum8(a);
      qd[i] = sum8(c);
    }
    uint16_t* yo = y + ((size_t)t * Hv + hv) * kDv;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float delta = (vs[r * kDv + grp + 32 * i] - kd[i]) * bt;
      const float yv = qd[i] + delta * kq;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sreg[i][j].x += kk[j].x * delta;
        sreg[i][j].y += kk[j].y * delta;
        sreg[i][j].z += kk[j].z * delta;
        sreg[i][j].w += kk[j].w * delta;
      }
      if (sub == i) yo[grp + 32 * i] = f2bf(yv);
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      *reinterpret_cast<float4*>(tile + (grp + 32 * i) * kDk + 4 * (sub + 8 * j)) = sreg[i][j];
}

size_t prefill_workspace_bytes(int R, int Hk, int total_tokens) {
  return carve(nullptr, R, Hk, total_tokens, nullptr);
}

template <int R>
static hipError_t launch_prefill_r(const PrefillArgs& a) {
  const int Hv = a.Hk * R;
  const int D = 2 * a.Hk * kDk + Hv * kDv;
  Workspace ws;
  carve(a.workspace, R, a.Hk, a.total_tokens, &ws);
  if (a.total_tokens > 0) {
    hipLaunchKernelGGL(prefill_conv_kernel, dim3(a.total_tokens, (D + 255) / 256), dim3(256), 0,
                       a.stream, a.conv, a.slot_ids, a.cu_seqlens, a.nseq, a.num_slots, D,
                       a.mixed, a.conv_w, ws.xc);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(prefill_conv_state_kernel, dim3(a.nseq, (D + 255) / 256), dim3(256), 0,
                     a.stream, a.conv, a.slot_ids, a.cu_seqlens, a.num_slots, D, a.total_tokens,
                     a.mixed);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.total_tokens > 0) {
    hipLaunchKernelGGL(prefill_prep_kernel<R>, dim3(a.total_tokens, a.Hk), dim3(256), 0,
                       a.stream, a.Hk, D, ws.xc, a.ab, a.A_log, a.dt_bias, ws.qn, ws.kn,
                       ws.beta, ws.g);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(prefill_seq_recurrence_kernel<R>, dim3(a.Hk, a.nseq), dim3(256 * R), 0,
                     a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, D,
                     a.total_tokens, ws.qn,
                     ws.kn, ws.xc, ws.g, ws.beta, a.y, a.status);
  return hipGetLastError();
}

hipError_t launch_prefill(const PrefillArgs& a) {
  switch (a.R) {
    case 1: return launch_prefill_r<1>(a);
    case 2: return launch_prefill_r<2>(a);
    case 4: return launch_prefill_r<4>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gdn
