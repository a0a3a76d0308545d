// gdn_attn.hip -- the attention layers' step on a paged KV cache
// (Qwen35Attention::forward_with_cache, qwen3_5.rs:377-455), for a packed
// batch of tokens from any number of sequences, each at its own position.
//
// The reference stacks per-sequence KV caches by zero-padding them to the
// longest and runs decode attention with no mask and one RoPE offset for the
// whole batch (mlx_executor.rs:57-88, qwen3_5.rs:410,443-447), so with B > 1
// a shorter sequence attends to padding and is rotated at the wrong
// position. Here every token carries its own sequence, position and KV page,
// keys are masked at each token's own position, and RoPE uses that position.
//
// Three launches per layer step (T tokens, Hq query heads, Hkv kv heads,
// G = Hq/Hkv query heads per kv head, head dim 256, pages of 64 tokens):
//   attn_prep_kernel    q, k rms-norm (qwen3_5.rs:399-407), partial RoPE
//                       (:411-417), K/V rows into the token's page
//   attn_block_kernel   one wave per worker of an even split of all
//                       (token group, kv head, 16-key block) work: scores and
//                       P.V on MFMA, online softmax, one partial per piece
//                       (scaled_dot_product_attention, :427-446)
//   attn_combine_kernel merge a token's pieces, output gate sigmoid(gate) *
//                       attn (:452-454), bf16 rows for o_proj
//
// Page layout. A page holds 64 positions of one layer: [2 (K, V)][Hkv][16384]
// bf16, each 16384-element tile stored in the order the MFMA operands are
// loaded, so that every load instruction of a wave reads 1 KiB (K) or 512 B
// (V) of contiguous memory (s = (kk/16) XOR (page % 4), the block's slot):
//   K (key kk, dim d): [s][d/32][(d/8)%4][kk%16][d%8]   -- A operand of
//       v_mfma_f32_16x16x32_bf16, rows = 16 keys, 32-deep k = dims
//   V (key kk, dim d): [s][d/16][(kk/4)%4][d%16][kk%4]  -- A operand of
//       v_mfma_f32_16x16x16_bf16, rows = 16 dims, 16-deep k = keys
#include "gdn_common.h"

namespace gdn {

namespace {

constexpr int kHd = 256;            // head dim = threads of the prep / combine work-groups
constexpr int kPage = 64;           // tokens per KV page
constexpr int kTile = kPage * kHd;  // elements of one page's K (or V) tile of one kv head
constexpr int kPartLd = 4 + kHd;    // partial row: m, l, 2 pad, 256 outputs (f32)
constexpr int kChunkBlocks = 24;    // 16-key blocks per chunk (384 keys, even): one partial each
static_assert(kChunkBlocks % 2 == 0, "chunks end after the second block of a pair");

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Slot of 16-key block b in page `page`: the four blocks' 8 KiB slots are
// XOR-swizzled by the page id, so that workers which start at the same block
// of different pages (and move in step) read different slots.
__device__ __forceinline__ int block_slot(int b, int page) { return b ^ (page & 3); }
__device__ __forceinline__ int k_off(int kk, int d, int page) {
  return (((block_slot(kk >> 4, page) * 8 + (d >> 5)) * 4 + ((d >> 3) & 3)) * 16 + (kk & 15)) * 8 +
         (d & 7);
}
__device__ __forceinline__ int v_off(int kk, int d, int page) {
  return (((block_slot(kk >> 4, page) * 16 + (d >> 4)) * 4 + ((kk >> 2) & 3)) * 16 + (d & 15)) * 4 +
         (kk & 3);
}

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

// 16-deep product: lane l holds row l%16, k = 4 (l/16) .. +3 of each operand
__device__ __forceinline__ f32x4 mfma16(uint2 a, uint2 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a),
                                                   __builtin_bit_cast(s16x4, b), c, 0, 0, 0);
}
__device__ __forceinline__ f32x4 mfma32(uint4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
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
    const int kk = pos & (kPage - 1);
    const size_t tile = ((size_t)page * 2 * Hkv + j) * kTile;
    pages[tile + k_off(kk, d, page)] = yb;  // K
    pages[tile + (size_t)Hkv * kTile + v_off(kk, d, page)] =
        v[(size_t)t * vs + (size_t)j * kHd + d];
    if (j == 0 && d == 0 && kk == 0) ptab[(size_t)slot * max_pages + pos / kPage] = page;
  }
}

// One wave per work-group; work-group w is worker w of P. The work is every
// (token group, kv head) segment's keys (segment s = group * Hkv + j) cut at
// fixed points into chunks of kChunkBlocks 16-key blocks; the flat list of
// all chunks, in segment order, goes to the workers in equal runs of k
// (worker w: chunks [w k, (w+1) k)), which may span several segments. Every
// chunk writes its own partial, so a token's result depends only on its own
// keys: the same in any batch, and when a prompt's tokens are grouped
// differently.
//
// A token group is up to 16/G consecutive tokens of one sequence: the 16
// columns of the MFMA tiles are (token, query head) pairs, column c = token
// c / G of the group, head j G + c % G. Per 16-key block:
//   S^T (16 keys x 16 columns) = K_blk (16 x 256) . Q^T (256 x 16): 8 MFMAs,
//     K straight from the page, Q^T loaded once per piece;
//   online softmax per column in the log2 domain (keys past the column's
//     token position masked to -inf; a wave-uniform branch rescales the
//     accumulators only when some column's running max grows);
//   O^T (256 dims x 16 columns) += V^T_blk . P^T: three 16-deep MFMAs per
//     16 dims, against P split into bf16 hi, mid and lo parts (together P's
////     24 significant bits: the products are those of float32 P). The score
//     accumulator of lane l holds keys 4 (l/16) .. +3 of column l%16: the B
//     operand layout as it is. (The O accumulators only
//     ever see the 16-deep opcode and the score accumulator only the 32-deep
//     one.)
// The next block's K and V are loaded while the current one computes, across
// chunk boundaries within a segment. V of keys past the group's last
// position is zeroed before use (those rows of a page may hold anything).
//
// Schedule tables (int32, built by the host for the step):
//   grp[NG][4]  first token, tokens, first position, sequence slot
//   seg[NS][4]  first chunk (= its partial), chunks, -, -
//   wseg[P]     segment of the worker's first chunk
// Partials [chunks][16][kPartLd] f32: running max (log2 domain), sum, output.
template <int G, bool STREAM>
__global__ __launch_bounds__(64, 2) void attn_block_kernel(
    const uint16_t* __restrict__ q_rot, int Hq, int Hkv, const int32_t* __restrict__ grp,
    const int32_t* __restrict__ seg, const int32_t* __restrict__ wseg, int NC, int k,
    const int32_t* __restrict__ ptab, int max_pages, const uint16_t* __restrict__ pages,
    float scale_log2, float* __restrict__ part) {
  static_assert(16 % G == 0, "whole tokens per 16 columns");
  __shared__ u32x4 qlds[8][64];  // this wave's Q^T operand
  const int w = blockIdx.x, lane = threadIdx.x;
  const int g4 = lane >> 4, c = lane & 15;
  const int gw1 = min(NC, (w + 1) * k);
  int g = w * k;  // next chunk
  int s = wseg[w];
  const size_t page_stride = (size_t)2 * Hkv * kTile;
  const size_t v_shift = (size_t)Hkv * kTile;
  while (g < gw1) {
    const int gi = s / Hkv, j = s - gi * Hkv;
    const int t0 = grp[4 * gi], ntok = grp[4 * gi + 1], pos0 = grp[4 * gi + 2],
              slot = grp[4 * gi + 3];
    const int cs0 = seg[4 * s], nch = seg[4 * s + 1];
    const int nkeys = pos0 + ntok;  // the group's last position + 1
    const int nblk = (nkeys + 15) >> 4;
    const int gend = min(gw1, cs0 + nch);  // this worker's chunks of the segment: [g, gend)
    const int kb0 = (g - cs0) * kChunkBlocks;
    const int kb1 = min(nblk, (gend - cs0) * kChunkBlocks);
    const int ctok = c / G;
    const bool cvalid = ctok < ntok;
    const int cpos = cvalid ? pos0 + ctok : -1;  // keys <= cpos are attended
    // Q^T: lane l holds column c, dims 32 ks + 8 g4 .. +7, kept in LDS
    {
      const uint4* qsrc = reinterpret_cast<const uint4*>(
          q_rot + ((size_t)(t0 + (cvalid ? ctok : 0)) * Hq + j * G + c % G) * kHd + 8 * g4);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const uint4 q = cvalid ? qsrc[4 * ks] : make_uint4(0, 0, 0, 0);
        qlds[ks][lane] = (u32x4){q.x, q.y, q.z, q.w};
      }
    }
    // the piece's page ids, one per lane (64 pages = 4096 keys per reload)
    const int32_t* prow = ptab + (size_t)slot * max_pages;
    const int npages = (nblk + 3) >> 2;
    int pbase = kb0 >> 2;
    int pid = pbase + lane < npages ? prow[pbase + lane] : 0;
    const uint16_t* kv_head = pages + (size_t)j * kTile;

    float m = -INFINITY, lsum = 0.f;
    f32x4 O[16];
#pragma unroll
    for (int db = 0; db < 16; ++db) O[db] = (f32x4){0.f, 0.f, 0.f, 0.f};

    auto load = [&](int kb, uint4(&kf)[8], uint2(&vf)[16]) {
      int idx = (kb >> 2) - pbase;
      if (idx >= 64) {  // wave-uniform: the next 64 page ids
        pbase += 64;
        idx -= 64;
        pid = pbase + lane < npages ? prow[pbase + lane] : 0;
      }
      const int page = __builtin_amdgcn_readlane(pid, idx);
      const uint16_t* kt =
          kv_head + (size_t)page * page_stride + (size_t)block_slot(kb & 3, page) * 4096;
      // STREAM (each block read about once in the step): non-temporal loads
      // stream past the caches; otherwise plain loads keep the blocks that
      // later token groups of the same prompt read again
      const u32x4* ksrc = reinterpret_cast<const u32x4*>(kt) + lane;
      const u32x2* vsrc = reinterpret_cast<const u32x2*>(kt + v_shift) + lane;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        const u32x4 x = STREAM ? __builtin_nontemporal_load(ksrc + 64 * ks) : ksrc[64 * ks];
        kf[ks] = make_uint4(x[0], x[1], x[2], x[3]);
      }
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        const u32x2 x = STREAM ? __builtin_nontemporal_load(vsrc + 64 * db) : vsrc[64 * db];
        vf[db] = make_uint2(x[0], x[1]);
      }
    };

    auto compute = [&](int kb, const uint4(&kf)[8], uint2(&vf)[16]) {
      f32x4 S = {0.f, 0.f, 0.f, 0.f};
      // Q^T is re-read from LDS for every block rather than held in registers:
      // an empty asm with a memory clobber keeps the compiler from hoisting
      // the reads (a volatile read would also drain the memory counters).
      asm volatile("" ::: "memory");
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) S = mfma32(kf[ks], qlds[ks][lane], S);
      const int key0 = 16 * kb + 4 * g4;  // this lane's keys key0 .. key0 + 3
      float x[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) x[r] = key0 + r <= cpos ? S[r] * scale_log2 : -INFINITY;
      float bm = fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3]));
      bm = fmaxf(bm, __shfl_xor(bm, 16, 64));
      bm = fmaxf(bm, __shfl_xor(bm, 32, 64));
      const float mnew = fmaxf(m, bm);
      if (__any(mnew > m)) {
        const float corr = mnew > m ? exp2f(m - mnew) : 1.0f;  // m = -inf: 0
        lsum *= corr;
#pragma unroll
        for (int db = 0; db < 16; ++db) O[db] *= corr;
        m = mnew;
      }
      const float mref = m == -INFINITY ? 0.f : m;
      float p[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) p[r] = exp2f(x[r] - mref);  // masked: exp2(-inf) = 0
      lsum += (p[0] + p[1]) + (p[2] + p[3]);
      // p = hi + mid + lo exactly: each part takes the next 8 significant bits
      uint32_t hi[4], mid[4], lo[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        hi[r] = f2bf(p[r]);
        const float r1 = p[r] - bf2f((uint16_t)hi[r]);
        mid[r] = f2bf(r1);
        lo[r] = f2bf(r1 - bf2f((uint16_t)mid[r]));
      }
      const uint2 ph = make_uint2(hi[0] | hi[1] << 16, hi[2] | hi[3] << 16);
      const uint2 pm = make_uint2(mid[0] | mid[1] << 16, mid[2] | mid[3] << 16);
      const uint2 pl = make_uint2(lo[0] | lo[1] << 16, lo[2] | lo[3] << 16);
      if (key0 + 3 >= nkeys) {  // rows past the group's last key: zero
        const uint32_t m0 = (key0 < nkeys ? 0xffffu : 0u) | (key0 + 1 < nkeys ? 0xffff0000u : 0u);
        const uint32_t m1 =
            (key0 + 2 < nkeys ? 0xffffu : 0u) | (key0 + 3 < nkeys ? 0xffff0000u : 0u);
#pragma unroll
        for (int db = 0; db < 16; ++db) {
          vf[db].x &= m0;
          vf[db].y &= m1;
        }
      }
#pragma unroll
      for (int db = 0; db < 16; ++db) {
        O[db] = mfma16(vf[db], ph, O[db]);
        O[db] = mfma16(vf[db], pm, O[db]);
        O[db] = mfma16(vf[db], pl, O[db]);
      }
    };

    // the partial of the chunk that block kb ends, then a fresh state
    auto flush = [&](int kb) {
      const float l4 = lsum + __shfl_xor(lsum, 16, 64);
      const float lt = l4 + __shfl_xor(l4, 32, 64);
      if (cvalid) {
        float* pr = part + ((size_t)(cs0 + kb / kChunkBlocks) * 16 + c) * kPartLd;
        if (g4 == 0) {
          pr[0] = m;
          pr[1] = lt;
        }
#pragma unroll
        for (int db = 0; db < 16; ++db)
          *reinterpret_cast<float4*>(pr + 4 + 16 * db + 4 * g4) =
              make_float4(O[db][0], O[db][1], O[db][2], O[db][3]);
      }
      m = -INFINITY;
      lsum = 0.f;
#pragma unroll
      for (int db = 0; db < 16; ++db) O[db] = (f32x4){0.f, 0.f, 0.f, 0.f};
    };

    uint4 kA[8], kB[8];
    uint2 vA[16], vB[16];
    load(kb0, kA, vA);
    // kb0 and the chunk size are even, so a chunk ends inside the range only
    // after the second block of a pair; the range's own end is flushed after.
    // Every pass issues its loads (an index past the range repeats the last
    // block), so the vector-memory counter waits for the block being
    // computed with the next one still in flight.
    for (int kb = kb0; kb < kb1; kb += 2) {
      load(min(kb + 1, kb1 - 1), kB, vB);
      compute(kb, kA, vA);
      if (kb + 1 >= kb1) break;
      load(min(kb + 2, kb1 - 1), kA, vA);
      compute(kb + 1, kB, vB);
      if ((kb + 2) % kChunkBlocks == 0 && kb + 2 < kb1) flush(kb + 1);
    }
    flush(kb1 - 1);
    g = gend;
    ++s;
  }
}

// grid (T, Hq), block 256: out[t, hq 256 + d] = bf16(bf16(o) *
// bf16(sigmoid(gate))) with o the normalised merge of the token's pieces for
// query head hq; gate is the second half of the head's q_proj outputs.
// tokseg[t] = the token's group, tokseg[T + t] = its first column. The 256
// threads first take the pieces' maxima, then work as 8 groups of 32 over the
// pieces (group i: pieces i, i + 8, ...; a thread 8 output dimensions), and
// the groups' sums meet in LDS, in a fixed order.
template <int G>
__global__ __launch_bounds__(kHd) void attn_combine_kernel(
    const float* __restrict__ part, const int32_t* __restrict__ tokseg,
    const int32_t* __restrict__ seg, int T, int Hkv, const uint16_t* __restrict__ q_full,
    int64_t qs, uint16_t* __restrict__ out, int64_t os) {
  __shared__ float red[8][kHd];
  __shared__ float redl[8];
  __shared__ float redm[4];
  const int t = blockIdx.x, hq = blockIdx.y, tid = threadIdx.x;
  const int j = hq / G, g = hq - j * G;
  const int s = tokseg[t] * Hkv + j;
  const int p0 = seg[4 * s], np = seg[4 * s + 1];
  const float* pc = part + ((size_t)p0 * 16 + tokseg[T + t] + g) * kPartLd;
  constexpr size_t kStride = (size_t)16 * kPartLd;  // consecutive pieces
  float mx = -INFINITY;
  for (int i = tid; i < np; i += kHd) mx = fmaxf(mx, pc[i * kStride]);
  mx = wave_max(mx);
  if ((tid & 63) == 0) redm[tid >> 6] = mx;
  __syncthreads();
  const float M = fmaxf(fmaxf(redm[0], redm[1]), fmaxf(redm[2], redm[3]));
  const int grp = tid >> 5, d8 = 8 * (tid & 31);
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float L = 0.f;
#pragma unroll 4
  for (int i = grp; i < np; i += 8) {
    const float* ps = pc + i * kStride;
    const float e = exp2f(ps[0] - M);  // a piece with no key of this token: 0
    L = fmaf(ps[1], e, L);
    const float4 a = *reinterpret_cast<const float4*>(ps + 4 + d8);
    const float4 b = *reinterpret_cast<const float4*>(ps + 8 + d8);
    acc[0] = fmaf(a.x, e, acc[0]);
    acc[1] = fmaf(a.y, e, acc[1]);
    acc[2] = fmaf(a.z, e, acc[2]);
    acc[3] = fmaf(a.w, e, acc[3]);
    acc[4] = fmaf(b.x, e, acc[4]);
    acc[5] = fmaf(b.y, e, acc[5]);
    acc[6] = fmaf(b.z, e, acc[6]);
    acc[7] = fmaf(b.w, e, acc[7]);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) red[grp][d8 + k] = acc[k];
  if ((tid & 31) == 0) redl[grp] = L;
  __syncthreads();
  float A = 0.f, Lt = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    A += red[i][tid];
    Lt += redl[i];
  }
  const float o = rbf(A / Lt);
  const float gate = bf2f(q_full[(size_t)t * qs + (size_t)hq * 2 * kHd + kHd + tid]);
  out[(size_t)t * os + (size_t)hq * kHd + tid] = f2bf(o * rbf(sigmoid_f32(gate)));
}

// grid (pages of the sequence, Hkv, 2), block 256: a sequence's cached K (z =
// 0) or V (z = 1) rows of one layer into dst [Hkv][len][256].
__global__ __launch_bounds__(kHd) void kv_gather_kernel(const uint16_t* __restrict__ pages,
                                                       const int32_t* __restrict__ prow, int Hkv,
                                                       int64_t len, uint16_t* __restrict__ k_out,
                                                       uint16_t* __restrict__ v_out) {
  const int p = blockIdx.x, j = blockIdx.y, isv = blockIdx.z, d = threadIdx.x;
  uint16_t* dst = isv ? v_out : k_out;
  if (!dst) return;
  const int page = prow[p];
  const uint16_t* tile = pages + ((size_t)page * 2 * Hkv + (size_t)isv * Hkv + j) * kTile;
  for (int kk = 0; kk < kPage; ++kk) {
    const int64_t pos = (int64_t)p * kPage + kk;
    if (pos >= len) break;
    dst[((size_t)j * len + pos) * kHd + d] = tile[isv ? v_off(kk, d, page) : k_off(kk, d, page)];
  }
}

size_t attn_part_offset(int T, int Hq) { return ((size_t)T * Hq * kHd * 2 + 255) & ~(size_t)255; }

size_t attn_workspace_bytes(int T, int Hq, int64_t chunks) {
  return attn_part_offset(T, Hq) + (size_t)chunks * 16 * kPartLd * sizeof(float);
}

int attn_chunk_blocks() { return kChunkBlocks; }

hipError_t launch_attn(const AttnArgs& a) {
  if (a.T <= 0) return hipSuccess;
  const int G = a.Hq / a.Hkv;
  uint16_t* q_rot = static_cast<uint16_t*>(a.workspace);
  float* part =
      reinterpret_cast<float*>(static_cast<char*>(a.workspace) + attn_part_offset(a.T, a.Hq));
  hipLaunchKernelGGL(attn_prep_kernel, dim3(a.T, a.Hq + a.Hkv), dim3(kHd), 0, a.stream, a.q_full,
                     a.qs, a.k, a.ks, a.v, a.vs, a.q_norm_w, a.k_norm_w, a.eps, a.rot_dim,
                     a.log2_base, a.Hq, a.Hkv, a.meta, a.T, a.ptab, a.max_pages, a.pages, q_rot);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const float scale_log2 = 1.4426950408889634f / sqrtf((float)kHd);  // log2(e) / sqrt(256)
  auto blocks = [&](auto kern) {
    hipLaunchKernelGGL(kern, dim3(a.P), dim3(64), 0, a.stream, q_rot, a.Hq, a.Hkv, a.grp, a.seg,
                       a.wseg, a.NC, a.kpw, a.ptab, a.max_pages, a.pages, scale_log2, part);
  };
  if (G == 8) {
    if (a.stream_keys)
      blocks(attn_block_kernel<8, true>);
    else
      blocks(attn_block_kernel<8, false>);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<8>), dim3(a.T, a.Hq), dim3(kHd), 0, a.stream, part,
                       a.tokseg, a.seg, a.T, a.Hkv, a.q_full, a.qs, a.out, a.os);
  } else if (G == 4) {
    if (a.stream_keys)
      blocks(attn_block_kernel<4, true>);
    else
      blocks(attn_block_kernel<4, false>);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL((attn_combine_kernel<4>), dim3(a.T, a.Hq), dim3(kHd), 0, a.stream, part,
                       a.tokseg, a.seg, a.T, a.Hkv, a.q_full, a.qs, a.out, a.os);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_kv_gather(const uint16_t* pages, const int32_t* prow, int Hkv, int64_t len,
                            uint16_t* k_out, uint16_t* v_out, hipStream_t s) {
  if (len <= 0) return hipSuccess;
  const int np = (int)((len + kPage - 1) / kPage);
  hipLaunchKernelGGL(kv_gather_kernel, dim3(np, Hkv, 2), dim3(kHd), 0, s, pages, prow, Hkv, len,
                     k_out, v_out);
  return hipGetLastError();
}

}  // namespace gdn
