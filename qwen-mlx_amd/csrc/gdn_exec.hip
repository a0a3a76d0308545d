// gdn_exec.hip -- the small kernels of the executor's model body around the
// GDN layers: token embedding rows, residual add + rms-norm, greedy pick.
// All three are row-parallel and HBM/latency bound (a few KB per row).
#include <climits>

#include "gdn_common.h"

namespace gdn {

namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxHiddenPerThread = 16;  // hidden <= 4096
constexpr int kMaxSlices = 8;            // K slices of a deferred projection (K <= 4096 in 512s)

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
//   h = bf16(h + d)   (skipped when d and dp are null)
// With dp, d is the bf16 rounding of the f32 sum of nslice partial rows
// dp[(sl * 64 + row) * npad + c], added in slice order: the value the
// projection's own slice-sum kernel would have stored, so the result is
// bit-identical to the two-launch form.
//   hn = bf16(w * bf16(h * rsqrt(mean(h^2) + eps)))
// With EMB the row comes from the embedding table instead (h = table[tok[i]],
// written out; no add): the stack's first seam fused with the embedding.
// grid n, block 256; thread t owns the 8 elements from 8t + 2048j (16-byte
// accesses; hidden a multiple of 8, at most 4096). NS = nslice (0: d or no
// add), a template argument so that every slice's loads go out together; the
// norm weights are loaded with them.
template <int NS, bool EMB>
__global__ __launch_bounds__(kRowThreads) void add_norm_kernel(uint16_t* __restrict__ h,
                                                               const uint16_t* __restrict__ d,
                                                               const float* __restrict__ dp,
                                                               int npad, int hidden,
                                                               const uint16_t* __restrict__ w,
                                                               float eps,
                                                               uint16_t* __restrict__ hn,
                                                               const uint16_t* __restrict__ table,
                                                               const int32_t* __restrict__ tok,
                                                               int vocab,
                                                               uint16_t* __restrict__ xsp) {
  __shared__ float red[4];
  constexpr int J = kMaxHiddenPerThread / 8;
  const size_t row = (size_t)blockIdx.x * hidden;
  const uint16_t* src = h + row;
  if constexpr (EMB) src = table + (size_t)min(max(tok[blockIdx.x], 0), vocab - 1) * hidden;
  float v[J][8];
  uint4 wv[J];
  float ss = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = 8 * (threadIdx.x + kRowThreads * j);
    if (c < hidden) {
      wv[j] = *reinterpret_cast<const uint4*>(w + c);
      uint4 hv = *reinterpret_cast<const uint4*>(src + c);
      if constexpr (EMB) *reinterpret_cast<uint4*>(h + row + c) = hv;
      const uint32_t* hw = reinterpret_cast<const uint32_t*>(&hv);
      if (NS > 0 || d != nullptr) {
        uint32_t dw[4];
        if constexpr (NS > 0) {
          // every slice's loads first (one round trip), then the adds in slice order
          const float* src = dp + (size_t)blockIdx.x * npad + c;
          v4f p0[NS > 0 ? NS : 1], p1[NS > 0 ? NS : 1];
#pragma unroll
          for (int sl = 0; sl < NS; ++sl) {
            const float* ps = src + (size_t)sl * 64 * npad;
            p0[sl] = *reinterpret_cast<const v4f*>(ps);
            p1[sl] = *reinterpret_cast<const v4f*>(ps + 4);
          }
          v4f t0 = p0[0], t1 = p1[0];
#pragma unroll
          for (int sl = 1; sl < NS; ++sl) {
            t0 += p0[sl];
            t1 += p1[sl];
          }
          dw[0] = f2bf2(t0[0], t0[1]);
          dw[1] = f2bf2(t0[2], t0[3]);
          dw[2] = f2bf2(t1[0], t1[1]);
          dw[3] = f2bf2(t1[2], t1[3]);
        } else {
          const uint4 dv = *reinterpret_cast<const uint4*>(d + row + c);
          const uint32_t* dr = reinterpret_cast<const uint32_t*>(&dv);
#pragma unroll
          for (int e = 0; e < 4; ++e) dw[e] = dr[e];
        }
        uint32_t o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e)
          o[e] = f2bf2(bf_lo(hw[e]) + bf_lo(dw[e]), bf_hi(hw[e]) + bf_hi(dw[e]));
        hv = make_uint4(o[0], o[1], o[2], o[3]);
        *reinterpret_cast<uint4*>(h + row + c) = hv;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[j][2 * e] = bf_lo(hw[e]);
        v[j][2 * e + 1] = bf_hi(hw[e]);
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += v[j][e] * v[j][e];
    }
  }
  const float tot = block_sum(ss, red);
  const float rn = 1.0f / sqrtf(tot / (float)hidden + eps);
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int c = 8 * (threadIdx.x + kRowThreads * j);
    if (c < hidden) {
      const uint32_t* ww = reinterpret_cast<const uint32_t*>(&wv[j]);
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        o[e] = f2bf2(bf_lo(ww[e]) * rbf(v[j][2 * e] * rn), bf_hi(ww[e]) * rbf(v[j][2 * e + 1] * rn));
      *reinterpret_cast<uint4*>(hn + row + c) = make_uint4(o[0], o[1], o[2], o[3]);
      if (xsp) {  // the sum of the 64 columns of group c / 64 (8 threads), split in three
        float gs = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) gs += bf_lo(o[e]) + bf_hi(o[e]);
        gs += __shfl_xor(gs, 1, 64);
        gs += __shfl_xor(gs, 2, 64);
        gs += __shfl_xor(gs, 4, 64);
        if ((threadIdx.x & 7) == 0) {
          const int G = hidden >> 6, g = c >> 6;
          const uint16_t hi = f2bf(gs);
          const float r = gs - bf2f(hi);
          const uint16_t md = f2bf(r);
          const size_t o0 = (size_t)blockIdx.x * G + g;
          xsp[o0] = hi;
          xsp[(size_t)64 * G + o0] = md;
          xsp[(size_t)128 * G + o0] = f2bf(r - bf2f(md));
        }
      }
    }
  }
}

// Greedy pick: out[i] = the index of the largest logit of row i (bf16
// [n, ld]); ties go to the lowest index and NaN never wins (an all-NaN row
// gives 0). Two passes: chunks of kArgChunk logits per work-group (16-byte
// loads), then one wave per row over the chunk winners.
constexpr int kArgChunk = 8192;

__device__ __forceinline__ void better(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ __launch_bounds__(kRowThreads) void argmax_part_kernel(const uint16_t* __restrict__ logits,
                                                                  int64_t ld, int vocab, int nchunk,
                                                                  float* __restrict__ pv,
                                                                  int* __restrict__ pi) {
  __shared__ float bvs[4];
  __shared__ int bis[4];
  const int chunk = blockIdx.x, r = blockIdx.y;
  const uint16_t* row = logits + (size_t)r * ld;
  float bv = -INFINITY;
  int bi = INT_MAX;  // no candidate yet
#pragma unroll
  for (int k = 0; k < kArgChunk / (8 * kRowThreads); ++k) {
    const int e = chunk * kArgChunk + 8 * (k * kRowThreads + threadIdx.x);
    if (e < vocab) {  // vocab is a multiple of 8
      const uint4 q = *reinterpret_cast<const uint4*>(row + e);
      const uint32_t* qw = reinterpret_cast<const uint32_t*>(&q);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const float a = bf_lo(qw[u]), b = bf_hi(qw[u]);
        if (a > bv || (bi == INT_MAX && a == bv)) { bv = a; bi = e + 2 * u; }
        if (b > bv || (bi == INT_MAX && b == bv)) { bv = b; bi = e + 2 * u + 1; }
      }
    }
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    better(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
  const int wave = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bvs[wave] = bv;
    bis[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < 4; ++k) better(bv, bi, bvs[k], bis[k]);
    pv[(size_t)r * nchunk + chunk] = bv;
    pi[(size_t)r * nchunk + chunk] = bi;
  }
}

__global__ __launch_bounds__(64) void argmax_final_kernel(const float* __restrict__ pv,
                                                          const int* __restrict__ pi, int nchunk,
                                                          int32_t* __restrict__ out,
                                                          int32_t* __restrict__ out_host) {
  const int r = blockIdx.x;
  float bv = -INFINITY;
  int bi = INT_MAX;
  for (int c = threadIdx.x; c < nchunk; c += 64) {
    const float v = pv[(size_t)r * nchunk + c];
    const int i = pi[(size_t)r * nchunk + c];
    if (i != INT_MAX) better(bv, bi, v, i);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1)
    better(bv, bi, __shfl_xor(bv, off, 64), __shfl_xor(bi, off, 64));
  if (threadIdx.x == 0) {
    out[r] = bi == INT_MAX ? 0 : bi;
    if (out_host) out_host[r] = bi == INT_MAX ? 0 : bi;
  }
}

// dst[i, :] = src[idx[i], :] (the last row of each packed prompt). grid n,
// block 256.
__global__ __launch_bounds__(kRowThreads) void gather_rows_kernel(const uint16_t* __restrict__ src,
                                                                  const int32_t* __restrict__ idx,
                                                                  int hidden,
                                                                  uint16_t* __restrict__ dst) {
  const uint4* s = reinterpret_cast<const uint4*>(src + (size_t)idx[blockIdx.x] * hidden);
  uint4* d = reinterpret_cast<uint4*>(dst + (size_t)blockIdx.x * hidden);
  for (int c = threadIdx.x; c < hidden / 8; c += kRowThreads) d[c] = s[c];
}

hipError_t launch_gather_rows(const uint16_t* src, const int32_t* idx, int n, int hidden,
                              uint16_t* dst, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(gather_rows_kernel, dim3(n), dim3(kRowThreads), 0, s, src, idx, hidden, dst);
  return hipGetLastError();
}

hipError_t launch_embed(const uint16_t* table, const int32_t* tok, int n, int vocab, int hidden,
                        uint16_t* h, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(embed_kernel, dim3(n), dim3(kRowThreads), 0, s, table, tok, vocab, hidden, h);
  return hipGetLastError();
}

hipError_t launch_add_norm(uint16_t* h, const uint16_t* d, const QPartial* dp, int n, int hidden,
                           const uint16_t* w, float eps, uint16_t* hn, hipStream_t s,
                           uint16_t* xsplit) {
  if (n <= 0) return hipSuccess;
  if (hidden > kRowThreads * kMaxHiddenPerThread || hidden % 8) return hipErrorInvalidValue;
  const bool part = dp != nullptr && dp->nslice > 0;
  if (part && (n > 64 || dp->Npad < hidden || dp->Npad % 8 || dp->nslice > kMaxSlices))
    return hipErrorInvalidValue;
  if (xsplit && (n > 64 || hidden % 64)) return hipErrorInvalidValue;
  const float* pp = part ? dp->part : nullptr;
  const uint16_t* dd = part ? nullptr : d;
  const int np = part ? dp->Npad : 0;
  switch (part ? dp->nslice : 0) {
#define GDN_ADD_NORM(NS)                                                                          \
  case NS:                                                                                        \
    hipLaunchKernelGGL((add_norm_kernel<NS, false>), dim3(n), dim3(kRowThreads), 0, s, h, dd, pp, \
                       np, hidden, w, eps, hn, nullptr, nullptr, 0, xsplit);                      \
    break;
    GDN_ADD_NORM(0) GDN_ADD_NORM(1) GDN_ADD_NORM(2) GDN_ADD_NORM(3) GDN_ADD_NORM(4)
    GDN_ADD_NORM(5) GDN_ADD_NORM(6) GDN_ADD_NORM(7) GDN_ADD_NORM(8)
#undef GDN_ADD_NORM
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_embed_norm(const uint16_t* table, const int32_t* tok, int n, int vocab,
                             int hidden, const uint16_t* w, float eps, uint16_t* h, uint16_t* hn,
                             hipStream_t s, uint16_t* xsplit) {
  if (n <= 0) return hipSuccess;
  if (hidden > kRowThreads * kMaxHiddenPerThread || hidden % 8) return hipErrorInvalidValue;
  if (xsplit && (n > 64 || hidden % 64)) return hipErrorInvalidValue;
  hipLaunchKernelGGL((add_norm_kernel<0, true>), dim3(n), dim3(kRowThreads), 0, s, h, nullptr,
                     nullptr, 0, hidden, w, eps, hn, table, tok, vocab, xsplit);
  return hipGetLastError();
}

int argmax_chunks(int vocab) { return (vocab + kArgChunk - 1) / kArgChunk; }

hipError_t launch_argmax(const uint16_t* logits, int64_t ld, int n, int vocab, float* pv, int* pi,
                         int32_t* out, int32_t* out_host, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int nc = argmax_chunks(vocab);
  hipLaunchKernelGGL(argmax_part_kernel, dim3(nc, n), dim3(kRowThreads), 0, s, logits, ld, vocab,
                     nc, pv, pi);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(argmax_final_kernel, dim3(n), dim3(64), 0, s, pv, pi, nc, out, out_host);
  return hipGetLastError();
}

}  // namespace gdn
