// gdn_exec.hip -- the small kernels of the executor's model body around the
// GDN layers: token embedding rows, residual add + rms-norm, greedy pick.
// All three are row-parallel and HBM/latency bound (a few KB per row).
#include "gdn_common.h"

namespace gdn {

namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxHiddenPerThread = 16;  // hidden <= 4096

// Block-wide f32 sum (every thread gets the result); red holds 4 floats.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) red[wave] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

}  // namespace

// h[i, :] = table[tok[i], :] (token ids are checked on the host; clamped here
// so that no id can address outside the table). grid n, block 256.
__global__ __launch_bounds__(kRowThreads) void embed_kernel(const uint16_t* __restrict__ table,
                                                            const int32_t* __restrict__ tok,
                                                            int vocab, int hidden,
                                                            uint16_t* __restrict__ h) {
  const int i = blockIdx.x;
  const int t = min(max(tok[i], 0), vocab - 1);
  const uint4* src = reinterpret_cast<const uint4*>(table + (size_t)t * hidden);
  uint4* dst = reinterpret_cast<uint4*>(h + (size_t)i * hidden);
  for (int c = threadIdx.x; c < hidden / 8; c += kRowThreads) dst[c] = src[c];
}

// Residual add then rms-norm of one row (the decoder layer's
// `x + mixer(input_layernorm(x))` seam, qwen3_5.rs:729-739):
//   h = bf16(h + d)   (skipped when d is null)
//   hn = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))
// grid n, block 256; thread t owns elements t + 256 j.
__global__ __launch_bounds__(kRowThreads) void add_norm_kernel(uint16_t* __restrict__ h,
                                                               const uint16_t* __restrict__ d,
                                                               int hidden,
                                                               const uint16_t* __restrict__ w,
                                                               float eps,
                                                               uint16_t* __restrict__ hn) {
  __shared__ float red[4];
  const size_t row = (size_t)blockIdx.x * hidden;
  float v[kMaxHiddenPerThread];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < kMaxHiddenPerThread; ++j) {
    const int c = threadIdx.x + kRowThreads * j;
    v[j] = 0.f;
    if (c < hidden) {
      float x = bf2f(h[row + c]);
      if (d != nullptr) {
        x = rbf(x + bf2f(d[row + c]));
        h[row + c] = f2bf(x);
      }
      v[j] = x;
      ss += x * x;
    }
  }
  const float tot = block_sum(ss, red);
  const float rn = 1.0f / sqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < kMaxHiddenPerThread; ++j) {
    const int c = threadIdx.x + kRowThreads * j;
    if (c < hidden) hn[row + c] = f2bf(bf2f(w[c]) * rbf(v[j] * rn));
  }
}

// out[i] = the index of the largest logit of row i (bf16 [n, ld]); ties go
// to the lowest index and NaN never wins (an all-NaN row gives 0). grid n,
// block 256.
__global__ __launch_bounds__(kRowThreads) void argmax_kernel(const uint16_t* __restrict__ logits,
                                                             int64_t ld, int vocab,
                                                             int32_t* __restrict__ out) {
  __shared__ float bvs[4];
  __shared__ int bis[4];
  const uint16_t* row = logits + (size_t)blockIdx.x * ld;
  float bv = -INFINITY;
  int bi = vocab;  // no candidate yet
  for (int c = threadIdx.x; c < vocab; c += kRowThreads) {
    const float x = bf2f(row[c]);
    if (x > bv || (bi == vocab && x == bv)) {  // first -inf still counts
      bv = x;
      bi = c;
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const float ov = __shfl_xor(bv, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    if (ov > bv || (ov == bv && oi < bi)) {
      bv = ov;
      bi = oi;
    }
  }
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bvs[wave] = bv;
    bis[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k)
      if (bvs[k] > bv || (bvs[k] == bv && bis[k] < bi)) {
        bv = bvs[k];
        bi = bis[k];
      }
    out[blockIdx.x] = bi == vocab ? 0 : bi;
  }
}

hipError_t launch_embed(const uint16_t* table, const int32_t* tok, int n, int vocab, int hidden,
                        uint16_t* h, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(kRowThreads), 0, s, table, tok, vocab, hidden, h);
  return hipGetLastError();
}

hipError_t launch_add_norm(uint16_t* h, const uint16_t* d, int n, int hidden, const uint16_t* w,
                           float eps, uint16_t* hn, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  if (hidden > kRowThreads * kMaxHiddenPerThread) return hipErrorInvalidValue;
  hipLaunchKernelGGL(add_norm_kernel, dim3(n), dim3(kRowThreads), 0, s, h, d, hidden, w, eps, hn);
  return hipGetLastError();
}

hipError_t launch_argmax(const uint16_t* logits, int64_t ld, int n, int vocab, int32_t* out,
                         hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(argmax_kernel, dim3(n), dim3(kRowThreads), 0, s, logits, ld, vocab, out);
  return hipGetLastError();
}

}  // namespace gdn
