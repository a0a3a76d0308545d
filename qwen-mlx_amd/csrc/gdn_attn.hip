// gdn_attn.hip -- the attention layers' step on a paged KV cache
// (Qwen35Attention::forward_with_cache, qwen3_5.rs:377-455), for a packed
// batch of tokens from any number of sequences, each at its own position.
//
// The reference stacks per-sequence KV caches by zero-padding them to the
// longest and runs decode attention with no mask and one RoPE offset for the
// whole batch (mlx_executor.rs:57-88, qwen3_5.rs:410,443-447), so with B > 1
// a shorter sequence attends to padding and is rotated at the wrong
// position. Here every token carries its own sequence, position and KV page,
// keys are masked at the sequence's length, and RoPE uses the token's own
// position.
//
// Three launches per layer step (T tokens, Hq query heads, Hkv kv heads,
// G = Hq/Hkv query heads per kv head, head dim 256, pages of 64 tokens):
//   attn_prep_kernel    q, k rms-norm (qwen3_5.rs:399-407), partial RoPE
//                       (:411-417), K/V rows into the token's page
//   attn_split_kernel   per (token, kv head, 1024-key split): scores of the G
//                       query heads against the split's keys, online softmax,
//                       P.V (scaled_dot_product_attention, :427-446)
//   attn_combine_kernel merge the splits, output gate sigmoid(gate) * attn
//                       (:452-454), bf16 rows for o_proj
#include "gdn_common.h"

namespace gdn {

namespace {

constexpr int kHd = 256;          // head dim = threads per work-group
constexpr int kPage = 64;         // tokens per KV page
constexpr int kSplitKeys = 1024;  // keys per attn_split_kernel work-group

// Block-wide f32 sum over 256 threads (every thread gets the result).
__device__ __forceinline__ float block_sum256(float v, float* red) {
  v = wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  const float t = (red[0] + red[1]) + (red[2] + red[3]);
  __syncthreads();
  return t;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

}  // namespace

// grid (T, Hq + Hkv), block 256: thread d owns dimension d of one head of one
// token. Heads < Hq are query heads (the first 256 of the head's 512 q_proj
// outputs; the other 256 are its output gate), the rest kv heads. The token's
// page comes with the step metadata; the first token of a page also records
// it in the sequence's page table, which the attention kernels read.
__global__ __launch_bounds__(kHd) void attn_prep_kernel(
    const uint16_t* __restrict__ q_full, int64_t qs, const uint16_t* __restrict__ k, int64_t ks,
    const uint16_t* __restrict__ v, int64_t vs, const uint16_t* __restrict__ q_norm_w,
    const uint16_t* __restrict__ k_norm_w, float eps, int rot_dim, float log2_base, int Hq,
    int Hkv, const int32_t* __restrict__ meta, int T, int32_t* __restrict__ ptab, int max_pages,
    uint16_t* __restrict__ pages, uint16_t* __restrict__ q_rot) {
  __shared__ float red[4];
  __shared__ float xs[kHd];
  const int t = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  const int slot = meta[t], pos = meta[T + t], page = meta[2 * T + t];
  const bool isq = h < Hq;
  const int j = h - Hq;  // kv head
  float x;
  if (isq)
    x = bf2f(q_full[(size_t)t * qs + (size_t)h * 2 * kHd + d]);
  else
    x = bf2f(k[(size_t)t * ks + (size_t)j * kHd + d]);
  const float ss = block_sum256(x * x, red);
  const float rn = 1.0f / sqrtf(ss / (float)kHd + eps);
  const float w = bf2f(isq ? q_norm_w[d] : k_norm_w[d]);
  const float xn = rbf(w * rbf(x * rn));
  // RoPE, rotate-half form over the first rot_dim dimensions: pairs (i, i + rot_dim/2)
  xs[d] = xn;
  __syncthreads();
  float y = xn;
  const int half = rot_dim >> 1;
  if (d < rot_dim) {
    const int i = d < half ? d : d - half;
    const float inv_freq = exp2f(-(2.0f * (float)i / (float)rot_dim) * log2_base);
    float sn, cs;
    sincosf((float)pos * inv_freq, &sn, &cs);
    y = d < half ? xn * cs - xs[d + half] * sn : xs[d - half] * sn + xn * cs;
  }
  const uint16_t yb = f2bf(y);
  if (isq) {
    q_rot[((size_t)t * Hq + h) * kHd + d] = yb;
  } else {
    const size_t row = (((size_t)page * 2 * Hkv + j) * kPage + (pos & (kPage - 1))) * kHd;
    pages[row + d] = yb;                                                         // K
    pages[row + (size_t)Hkv * kPage * kHd + d] = v[(size_t)t * vs + (size_t)j * kHd + d];  // V
    if (j == 0 && d == 0 && (pos & (kPage - 1)) == 0) ptab[(size_t)slot * max_pages + pos / kPage] = page;
  }
}

// grid (T, Hkv, splits), block 256. Work-group (t, j, sp) takes keys
// [1024 sp, min(1024 (sp + 1), pos_t + 1)) of token t's sequence for the G
// query heads of kv head j: K and V pages staged in LDS (64 keys x 512 B
// each; K rows padded to 528 B so that the 64 lanes reading 64 different
// rows hit distinct banks), scores with the 64 keys on the lanes of a wave
// (wave w: query heads w G/4 .. w G/4 + G/4 - 1), online softmax per head,
// then P.V with thread d owning output dimension d. Writes the split's
// running max, sum and unnormalised output (f32) to part.
template <int G>
__global__ __launch_bounds__(kHd) void attn_split_kernel(
    const uint16_t* __restrict__ q_rot, int Hq, int Hkv, const int32_t* __restrict__ meta, int T,
    const int32_t* __restrict__ ptab, int max_pages, const uint16_t* __restrict__ pages,
    float scale, int nsplit_max, float* __restrict__ part) {
  static_assert(G % 4 == 0, "G/4 query heads per wave");
  constexpr int GW = G / 4;
  constexpr int KLD = kHd + 8;  // padded K row (bf16)
  __shared__ __align__(16) float q[G][kHd];
  __shared__ __align__(16) uint16_t Ks[kPage][KLD];
  __shared__ __align__(16) uint16_t Vs[kPage][kHd];
  __shared__ __align__(16) float p[G][kPage];
  __shared__ float corr[G];
  const int t = blockIdx.x, j = blockIdx.y, sp = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int slot = meta[t], pos = meta[T + t];
  const int nkeys = pos + 1;
  const int k0 = sp * kSplitKeys;
  if (k0 >= nkeys) return;
  const int k1 = min(k0 + kSplitKeys, nkeys);
#pragma unroll
  for (int g = 0; g < G; ++g) q[g][tid] = bf2f(q_rot[((size_t)t * Hq + j * G + g) * kHd + tid]);
  float m[GW], l[GW];
#pragma unroll
  for (int u = 0; u < GW; ++u) {
    m[u] = -INFINITY;
    l[u] = 0.f;
  }
  float acc[G];
#pragma unroll
  for (int g = 0; g < G; ++g) acc[g] = 0.f;
  const int32_t* prow = ptab + (size_t)slot * max_pages;
  for (int kb = k0; kb < k1; kb += kPage) {
    const int n = min(kPage, k1 - kb);
    const size_t base = ((size_t)prow[kb / kPage] * 2 * Hkv + j) * kPage * kHd;
    const uint4* ksrc = reinterpret_cast<const uint4*>(pages + base);
    const uint4* vsrc = reinterpret_cast<const uint4*>(pages + base + (size_t)Hkv * kPage * kHd);
    __syncthreads();  // the previous page's readers are done
#pragma unroll
    for (int r = 0; r < kPage * kHd / 8 / kHd; ++r) {  // 8 uint4 per thread per array
      const int e = tid + kHd * r;  // row e / 32, 16-byte chunk e % 32
      *reinterpret_cast<uint4*>(&Ks[e >> 5][8 * (e & 31)]) = ksrc[e];
      reinterpret_cast<uint4*>(&Vs[0][0])[e] = vsrc[e];
    }
    __syncthreads();
    // scores: lane = key, this wave's GW heads
    float s[GW];
#pragma unroll
    for (int u = 0; u < GW; ++u) s[u] = 0.f;
    const uint4* krow = reinterpret_cast<const uint4*>(&Ks[lane][0]);  // 528-byte rows
#pragma unroll 4
    for (int c = 0; c < kHd / 8; ++c) {
      const uint4 kv = krow[c];
      const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int u = 0; u < GW; ++u) {
        const float4 qa = *reinterpret_cast<const float4*>(&q[wave * GW + u][8 * c]);
        const float4 qb = *reinterpret_cast<const float4*>(&q[wave * GW + u][8 * c + 4]);
        s[u] = fmaf(qa.x, bf_lo(kw[0]), s[u]);
        s[u] = fmaf(qa.y, bf_hi(kw[0]), s[u]);
        s[u] = fmaf(qa.z, bf_lo(kw[1]), s[u]);
        s[u] = fmaf(qa.w, bf_hi(kw[1]), s[u]);
        s[u] = fmaf(qb.x, bf_lo(kw[2]), s[u]);
        s[u] = fmaf(qb.y, bf_hi(kw[2]), s[u]);
        s[u] = fmaf(qb.z, bf_lo(kw[3]), s[u]);
        s[u] = fmaf(qb.w, bf_hi(kw[3]), s[u]);
      }
    }
#pragma unroll
    for (int u = 0; u < GW; ++u) {
      const float sc = lane < n ? s[u] * scale : -INFINITY;
      const float mnew = fmaxf(m[u], wave_max(sc));
      const float pe = lane < n ? expf(sc - mnew) : 0.f;
      const float c = expf(m[u] - mnew);  // 0 for the first page (m = -inf)
      l[u] = l[u] * c + wave_sum(pe);
      m[u] = mnew;
      p[wave * GW + u][lane] = pe;
      if (lane == 0) corr[wave * GW + u] = c;
    }
    __syncthreads();
    // P.V: thread tid owns dimension tid of every query head
#pragma unroll
    for (int g = 0; g < G; ++g) acc[g] *= corr[g];
    // keys past n have p = 0 (their V rows may hold anything but are finite
    // or not, so they are skipped, four keys at a time up to n)
    for (int key = 0; key < n; key += 4) {
      float vv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) vv[e] = key + e < n ? bf2f(Vs[key + e][tid]) : 0.f;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float4 pp = *reinterpret_cast<const float4*>(&p[g][key]);
        acc[g] = fmaf(pp.x, vv[0], acc[g]);
        acc[g] = fmaf(pp.y, vv[1], acc[g]);
        acc[g] = fmaf(pp.z, vv[2], acc[g]);
        acc[g] = fmaf(pp.w, vv[3], acc[g]);
      }
    }
  }
  // partials [T][Hkv][nsplit_max][G][2 + 256]: m, l, then the output
  const size_t pb = (((size_t)t * Hkv + j) * nsplit_max + sp) * G * (2 + kHd);
#pragma unroll
  for (int g = 0; g < G; ++g) part[pb + (size_t)g * (2 + kHd) + 2 + tid] = acc[g];
  if (lane == 0) {
#pragma unroll
    for (int u = 0; u < GW; ++u) {
      part[pb + (size_t)(wave * GW + u) * (2 + kHd)] = m[u];
      part[pb + (size_t)(wave * GW + u) * (2 + kHd) + 1] = l[u];
    }
  }
}

// grid (T, Hkv), block 256: out[t, (j G + g) 256 + d] = bf16(bf16(o) *
// bf16(sigmoid(gate))) with o the normalised merge of the splits; gate is the
// second half of the head's q_proj outputs.
template <int G>
__global__ __launch_bounds__(kHd) void attn_combine_kernel(
    const float* __restrict__ part, const int32_t* __restrict__ meta, int T, int Hkv,
    int nsplit_max, const uint16_t* __restrict__ q_full, int64_t qs, uint16_t* __restrict__ out,
    int64_t os) {
  const int t = blockIdx.x, j = blockIdx.y, d = threadIdx.x;
  const int nkeys = meta[T + t] + 1;
  const int ns = (nkeys + kSplitKeys - 1) / kSplitKeys;
  const size_t pb = ((size_t)t * Hkv + j) * nsplit_max * G * (2 + kHd);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    float M = -INFINITY;
    for (int sp = 0; sp < ns; ++sp) M = fmaxf(M, part[pb + ((size_t)sp * G + g) * (2 + kHd)]);
    float L = 0.f, A = 0.f;
    for (int sp = 0; sp < ns; ++sp) {
      const float* ps = part + pb + ((size_t)sp * G + g) * (2 + kHd);
      const float e = expf(ps[0] - M);
      L = fmaf(ps[1], e, L);
      A = fmaf(ps[2 + d], e, A);
    }
    const int hq = j * G + g;
    const float o = rbf(A / L);
    const float gate = bf2f(q_full[(size_t)t * qs + (size_t)hq * 2 * kHd + kHd + d]);
    out[(size_t)t * os + (size_t)hq * kHd + d] = f2bf(o * rbf(sigmoid_f32(gate)));
  }
}

int attn_splits(int max_keys) { return (max_keys + kSplitKeys - 1) / kSplitKeys; }

size_t attn_workspace_bytes(int T, int Hq, int Hkv, int nsplit) {
  const size_t qrot = ((size_t)T * Hq * kHd * 2 + 255) & ~(size_t)255;
  const size_t part = (size_t)T * Hq * nsplit * (2 + kHd) * sizeof(float);
  return qrot + part;
}

hipError_t launch_attn(const AttnArgs& a) {
  if (a.T <= 0) return hipSuccess;
  const int G = a.Hq / a.Hkv;
  uint16_t* q_rot = static_cast<uint16_t*>(a.workspace);
  float* part = reinterpret_cast<float*>(static_cast<char*>(a.workspace) +
                                         (((size_t)a.T * a.Hq * kHd * 2 + 255) & ~(size_t)255));
  hipLaunchKernelGGL(attn_prep_kernel, dim3(a.T, a.Hq + a.Hkv), dim3(kHd), 0, a.stream, a.q_full,
                     a.qs, a.k, a.ks, a.v, a.vs, a.q_norm_w, a.k_norm_w, a.eps, a.rot_dim,
                     a.log2_base, a.Hq, a.Hkv, a.meta, a.T, a.ptab, a.max_pages, a.pages, q_rot);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const float scale = 1.0f / sqrtf((float)kHd);
  if (G == 8) {
    hipLaunchKernelGGL((attn_split_kernel<8>), dim3(a.T, a.Hkv, a.nsplit), dim3(kHd), 0, a.stream,
                       q_rot, a.Hq, a.Hkv, a.meta, a.T, a.ptab, a.max_pages, a.pages, scale,
                       a.nsplit, part);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<8>), dim3(a.T, a.Hkv), dim3(kHd), 0, a.stream, part,
                       a.meta, a.T, a.Hkv, a.nsplit, a.q_full, a.qs, a.out, a.os);
  } else if (G == 4) {
    hipLaunchKernelGGL((attn_split_kernel<4>), dim3(a.T, a.Hkv, a.nsplit), dim3(kHd), 0, a.stream,
                       q_rot, a.Hq, a.Hkv, a.meta, a.T, a.ptab, a.max_pages, a.pages, scale,
                       a.nsplit, part);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<4>), dim3(a.T, a.Hkv), dim3(kHd), 0, a.stream, part,
                       a.meta, a.T, a.Hkv, a.nsplit, a.q_full, a.qs, a.out, a.os);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace gdn
