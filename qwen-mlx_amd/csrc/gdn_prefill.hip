// gdn_prefill.hip -- varlen prefill of packed sequences (cu_seqlens).
//
// The reference runs prefill one sequence at a time (B=1) through
// GatedDeltaNet::forward_with_cache with S>1 (qwen3_5.rs:611-658): conv1d
// over [conv_state | x], silu, split, q/k rms-norm, gates, and one
// gated_delta_kernel launch with T=S (metal_gdn.rs:37). Here any number of
// sequences share the launches, each addressed by its slot:
//   1. qkv_kernel        conv + silu, q/k rms-norm -> qn/kn/vc, gates -> beta, lg
//   2. conv_state_kernel last K-1 rows of [conv_state | x] -> slot
//   3. chunk_kernel      chunked WY-form recurrence on bf16 MFMA
// Workspace layout (each region 256-byte aligned):
//   qn [T,Hk,Dk] bf16 | kn [T,Hk,Dk] bf16 | vc [T,Hv,Dv] bf16 | beta [T,Hv] bf16 | lg [T,Hv] f32

#include <mutex>

#include "gdn_common.h"

namespace gdn {

namespace {

constexpr float kQNormW = 0.0078125f;
constexpr float kKNormW = 0.08837890625f;
constexpr float kNormEps = 1e-6f;
constexpr int kTT = 64;  // tokens per qkv_kernel work-group

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Workspace {
  uint16_t* qn;
  uint16_t* kn;
  uint16_t* vc;
  uint16_t* beta;
  float* lg;
};

size_t carve(void* base, int R, int Hk, int T, Workspace* w) {
  const int Hv = Hk * R;
  size_t off = 0;
  char* p = static_cast<char*>(base);
  auto take = [&](size_t bytes) {
    void* r = p ? p + off : nullptr;
    off += align256(bytes);
    return r;
  };
  Workspace ws;
  ws.qn = static_cast<uint16_t*>(take((size_t)T * Hk * kDk * 2));
  ws.kn = static_cast<uint16_t*>(take((size_t)T * Hk * kDk * 2));
  ws.vc = static_cast<uint16_t*>(take((size_t)T * Hv * kDv * 2));
  ws.beta = static_cast<uint16_t*>(take((size_t)T * Hv * 2));
  ws.lg = static_cast<float*>(take((size_t)T * Hv * 4));
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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// The sigmoid of the conv activations on the hardware exp2 and reciprocal
// (v_exp_f32, v_rcp_f32; ~2 ulp instead of the ~1 ulp of expf and an IEEE
// divide). Its result is rounded to bf16 next, so the two forms differ only
// where the exact value lies within a few f32 ulp of a bf16 rounding
// boundary, by one bf16 ulp.
__device__ __forceinline__ float sigmoid_fast(float x) {
  const float e = __builtin_amdgcn_exp2f(-fabsf(x) * 1.4426950408889634f);
  const float y = __builtin_amdgcn_rcpf(1.0f + e);
  return x < 0.0f ? 1.0f - y : y;
}

}  // namespace

// 1. Per (64-token tile, 128-channel head) of mixed_qkv; heads 0..Hk-1 are q,
// Hk..2Hk-1 are k, the rest v (the channel order of the qkv projection):
//   conv1d + silu (qwen3_5.rs:617-623): c[t,ch] = silu(sum_k padded[t+k,ch] w[ch,k])
//     with padded = [slot conv state (K-1 rows) | x of the sequence]; f32
//     accumulation, one rounding to bf16;
//   q/k heads: rms-norm with the baked weights (qwen3_5.rs:627-633) -> qn, kn;
//   v heads: c -> vc, and the gates of that head (compiled_ops.rs:68-94):
//     beta = sigmoid(b), lg = log g = -exp(A_log) softplus(a + dt_bias).
// The 64 + K-1 input rows of the tile are staged in LDS once (one HBM read per
// element plus a 3-row halo); lane l of a 16-lane group owns channels 8l..8l+7
// of one token. grid (2Hk+Hv, ceil(T/64)), block 256.
template <int R>
__global__ __launch_bounds__(256) void prefill_qkv_kernel(
    const uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int nseq, int num_slots, int Hk, int T,
    const uint16_t* __restrict__ x, int64_t xs, const uint16_t* __restrict__ conv_w,
    const uint16_t* __restrict__ ab, int64_t abs_, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, uint16_t* __restrict__ qn, uint16_t* __restrict__ kn,
    uint16_t* __restrict__ vc, uint16_t* __restrict__ beta, float* __restrict__ lg) {
  constexpr int KH = kConvK - 1;
  __shared__ uint4 tile[kTT + KH][16];
  __shared__ int tok_st[kTT];    // first token of the token's sequence (clamped <= t)
  __shared__ int tok_slot[kTT];  // slot of that sequence, -1 if invalid
  const int head = blockIdx.x, t0 = blockIdx.y * kTT;
  const int Hv = Hk * R;
  const int D = (2 * Hk + Hv) * kDk;
  const int tid = threadIdx.x;
  const size_t hcol = (size_t)head * kDk;
  for (int e = tid; e < (kTT + KH) * 16; e += 256) {
    const int r = e >> 4, c = e & 15, u = t0 - KH + r;
    u32x4 v = {0u, 0u, 0u, 0u};
    if (u >= 0 && u < T)
      v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(x + (size_t)u * xs + hcol) + c);
    tile[r][c] = make_uint4(v.x, v.y, v.z, v.w);
  }
  if (tid < kTT) {
    const int t = t0 + tid;
    int st = t, sl = -1;
    if (t < T) {
      const int s = seq_of(cu, nseq, t);
      st = min(max(cu[s], 0), t);
      sl = slot_ids[s];
      if ((unsigned)sl >= (unsigned)num_slots) sl = -1;  // flagged by the chunk kernel
    }
    tok_st[tid] = st;
    tok_slot[tid] = sl;
  }
  const int l = tid & 15;
  // conv weights of channels 8l..8l+7: [8][K] bf16 = 4 x uint4
  float wk[8][kConvK];
  {
    const uint4* wp = reinterpret_cast<const uint4*>(conv_w + (hcol + 8 * l) * kConvK);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint4 v = wp[q];
      const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        wk[2 * q + h][0] = bf_lo(wd[2 * h]);
        wk[2 * q + h][1] = bf_hi(wd[2 * h]);
        wk[2 * q + h][2] = bf_lo(wd[2 * h + 1]);
        wk[2 * q + h][3] = bf_hi(wd[2 * h + 1]);
      }
    }
  }
  __syncthreads();
  const bool isq = head < Hk, isk = !isq && head < 2 * Hk;
#pragma unroll
  for (int it = 0; it < kTT / 16; ++it) {
    const int i = (tid >> 4) + 16 * it, t = t0 + i;
    const int st = tok_st[i];
    uint32_t win[kConvK][4];  // taps t-K+1..t, channels 8l..8l+7 as bf16 pairs
    if (t - KH >= st) {
#pragma unroll
      for (int k = 0; k < kConvK; ++k) {
        const uint4 v = tile[i + k][l];
        win[k][0] = v.x; win[k][1] = v.y; win[k][2] = v.z; win[k][3] = v.w;
      }
    } else {  // within K-1 tokens of the sequence start: taps before it come from the conv state
      const int sl = tok_slot[i];
#pragma unroll
      for (int k = 0; k < kConvK; ++k) {
        const int u = t + k - KH;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (u >= st)
          v = tile[i + k][l];
        else if (sl >= 0)  // conv state row u - st + K-1
          v = *reinterpret_cast<const uint4*>(conv + ((size_t)sl * KH + (u - st + KH)) * D + hcol + 8 * l);
        win[k][0] = v.x; win[k][1] = v.y; win[k][2] = v.z; win[k][3] = v.w;
      }
    }
    // bf16 x bf16 products are exact in f32, so the fused multiply-adds equal
    // the sequential f32 accumulation of the products.
    float cv[8];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
      float a0 = 0.f, a1 = 0.f;
#pragma unroll
      for (int k = 0; k < kConvK; ++k) {
        a0 = fmaf(bf_lo(win[k][h]), wk[2 * h][k], a0);
        a1 = fmaf(bf_hi(win[k][h]), wk[2 * h + 1][k], a1);
      }
      rbf2(a0, a1);
      float s0 = sigmoid_fast(a0), s1 = sigmoid_fast(a1);
      rbf2(s0, s1);
      float c0 = a0 * s0, c1 = a1 * s1;
      rbf2(c0, c1);
      cv[2 * h] = c0;
      cv[2 * h + 1] = c1;
    }
    uint32_t o[4];
    uint16_t* dst;
    if (isq || isk) {
      float ss = 0.f;
#pragma unroll
      for (int c = 0; c < 8; ++c) ss = fmaf(cv[c], cv[c], ss);
#pragma unroll
      for (int m = 1; m < 16; m <<= 1) ss += __shfl_xor(ss, m, 64);
      const float rn = 1.0f / sqrtf(ss / (float)kDk + kNormEps);
      const float wn = isq ? kQNormW : kKNormW;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        float n0 = cv[2 * h] * rn, n1 = cv[2 * h + 1] * rn;
        rbf2(n0, n1);
        o[h] = f2bf2(wn * n0, wn * n1);
      }
      dst = (isq ? qn : kn) + ((size_t)t * Hk + (isq ? head : head - Hk)) * kDk;
    } else {
#pragma unroll
      for (int h = 0; h < 4; ++h) o[h] = f2bf2(cv[2 * h], cv[2 * h + 1]);
      dst = vc + ((size_t)t * Hv + (head - 2 * Hk)) * kDv;
    }
    if (t < T) reinterpret_cast<uint4*>(dst)[l] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (!isq && !isk && tid < kTT && t0 + tid < T) {
    const int t = t0 + tid, h = head - 2 * Hk;
    const float braw = bf2f(ab[(size_t)t * abs_ + h]);
    const float araw = bf2f(ab[(size_t)t * abs_ + Hv + h]);
    beta[(size_t)t * Hv + h] = f2bf(sigmoid_f32(braw));
    // log of the decay multiplier g = exp(lg) (compiled_ops.rs:36-43); the
    // naive softplus overflows to inf for a+dt_bias >~ 88 (g = 0), clamped so
    // that differences of cumulative sums stay finite (exp(-1e4) == 0 in f32)
    const float sp = logf(expf(araw + dt_bias[h]) + 1.0f);
    lg[(size_t)t * Hv + h] = fmaxf(-(expf(A_log[h]) * sp), -1.0e4f);
  }
}

// 2. new conv state = last K-1 rows of padded (qwen3_5.rs:618-619).
// Runs after (1) has read the old rows. grid (nseq, D/256), block 256. Also
// checks cu_seqlens (cu[0] = 0, non-decreasing, cu[nseq] = T), latching
// GDN_FLAG_BAD_SEQLENS; every kernel clamps the bounds it reads either way.
__global__ __launch_bounds__(256) void prefill_conv_state_kernel(
    uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int nseq, int num_slots, int D, int T,
    const uint16_t* __restrict__ x, int64_t xs, uint32_t* __restrict__ status) {
  const int s = blockIdx.x;
  const int ch = blockIdx.y * 256 + threadIdx.x;
  if (blockIdx.y == 0 && threadIdx.x == 0) {
    const int a = cu[s], b = cu[s + 1];
    if ((s == 0 && a != 0) || b < a || b > T || (s == nseq - 1 && b != T))
      flag_status(status, GDN_FLAG_BAD_SEQLENS);
  }
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
                                      : x[(size_t)(st + p - (kConvK - 1)) * xs + ch];
    cs[(size_t)j * D + ch] = v;
  }
}

// 3. Chunked (WY form) recurrence, one work-group of 512 threads (8 waves) per
// (sequence, value head), walking the sequence's chunks of kC = 64 tokens. With G the cumulative log decay inside a chunk and S
// ([Dv, Dk]) the state at the chunk start:
//   L_ij = beta_i (k_i.k_j) exp(G_i - G_j)   (j < i)
//   P_ij = (q_i.k_j) exp(G_i - G_j)          (j <= i)
//   R    = beta * (V - exp(G) * (K S^T))      per token row
//   (I + L) V' = R                            (block forward substitution)
//   O    = exp(G) * (Q S^T) + P V'
//   S^T <- exp(G_C) S^T + K^T (exp(G_C - G) * V')
// which equals the token-by-token recurrence of metal_gdn.rs:37-62.
//
// Work split: waves 0-3 form K K^T (token row block w) and invert its
// diagonal block, waves 4-7 form Q K^T; every other step runs wave-locally on
// the wave's own 16 state rows (dv block w), so a chunk needs three
// work-group barriers. The triangular solve works on V'
// directly, 16-token blocks: V'_I = D_I (R_I - sum_{j<I} L_Ij V'_j) with
// D_I = (I + L_II)^-1. A 16x16 MFMA accumulator holds row 4*(l/16) + r,
// column l%16 of its tile in register r of lane l, which is the B-operand
// layout of a 16-deep product: V' blocks and state tiles feed the next
// products without data movement. k and q are bf16 (exact operands); f32
// operands on the state path (S, L, D, R, V') are split into bf16 hi + lo
// parts (~16 mantissa bits). A product with a split operand, X.Bh + X.Bl, is
// one v_mfma_f32_16x16x32_bf16 whose 32-deep k axis holds, in each lane
// group's 8 slots, 4 k of the hi part then the same 4 k of the lo part, with
// the A fragment repeated (cat): the accumulator-layout registers are the B
// operand as they are. The state lives in MFMA accumulators (S^T tiles)
// across chunks. The next chunk's inputs are loaded into
// registers while the current chunk computes. Padded rows of a
// partial chunk have k = q = v = beta = 0 and log decay 0, so they change
// nothing.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kC = 64;
constexpr int kLdK = kDk + 8;  // bf16 [64][128] rows (272 B)
constexpr int kLdT = kC + 8;   // bf16 [*][64] rows (144 B)
constexpr int kLdD = 24;       // bf16 [16][16] blocks (48 B rows)

struct ChunkSmem {
  uint16_t K[kC][kLdK];      // k, token-major
  uint16_t KT[kDk][kLdT];    // k, dk-major
  uint16_t Q[kC][kLdK];      // q, token-major
  uint16_t V[kC][kLdK];      // v of the head, token-major
  uint16_t P[kC][kLdT];      // masked, decayed q.k
  uint16_t NLh[kC][kLdT];    // -L, bf16 hi part
  uint16_t NLl[kC][kLdT];    // -L, bf16 lo part
  float Ld[4][16][17];       // diagonal 16x16 blocks of L (f32)
  uint16_t Dh[4][16][kLdD];  // D_I = (I + L_II)^-1, hi
  uint16_t Dl[4][16][kLdD];  // lo
  float beta[kC], G[kC], eG[kC], dec_end[kC];  // G: cumulative log2 decay
  float ysq[kC][8];          // RMSNormGated: per token, each wave's sum of y^2
};

__device__ __forceinline__ f32x4 mfma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Operand fragments whose k runs contiguous in memory; they serve as A
// operands (rows = output rows) and as B operands (rows = output columns).
//   frag32: lane l takes row r0 + l%16, k = k0 + 8*(l/16) .. +7
//   frag16: lane l takes row r0 + l%16, k = k0 + 4*(l/16) .. +3
// A 16x16 accumulator tile holds row 4*(l/16) + r, column l%16 in register r:
// the frag16 layout of its transpose, i.e. a B operand with k = row.
__device__ __forceinline__ bf16x8 frag32(const uint16_t* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + (r0 + (lane & 15)) * ld + k0 + (lane >> 4) * 8);
}
__device__ __forceinline__ s16x4 frag16(const uint16_t* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const s16x4*>(base + (r0 + (lane & 15)) * ld + k0 + (lane >> 4) * 4);
}

__device__ __forceinline__ short bfbits(float x) { return (short)f2bf(x); }

// Two 4-element fragments as one 8-element MFMA operand. Every product of
// the kernel is a v_mfma_f32_16x16x32_bf16, a lone 16-deep term padded with
// zeros: accumulation chains that mixed it with v_mfma_f32_16x16x16_bf16
// (the result of one feeding the accumulator of the other) gave wrong results
// in testing, so no accumulator is ever shared between the two opcodes.
typedef short s16x8 __attribute__((ext_vector_type(8)));
constexpr s16x4 kZero4 = {0, 0, 0, 0};
__device__ __forceinline__ bf16x8 cat(s16x4 a, s16x4 b) {
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}

// K^T is stored with its token column XOR-swizzled by 8 * ((dk >> 3) & 7):
// the transposing 2-byte stores of one wave (16 dk rows 8 apart) then spread
// over the LDS banks, and a 4-token group stays contiguous and 8-byte aligned.
__device__ __forceinline__ int kt_col(int dk, int tok) { return tok ^ (((dk >> 3) & 7) << 3); }
__device__ __forceinline__ s16x4 frag16_kt(const uint16_t (*KT)[kC + 8], int r0, int k0, int lane) {
  const int row = r0 + (lane & 15);
  return *reinterpret_cast<const s16x4*>(&KT[row][kt_col(row, k0 + (lane >> 4) * 4)]);
}

// f32 tile -> bf16 hi + lo (hi + lo carries ~16 mantissa bits of x)
__device__ __forceinline__ void split4(const f32x4& x, s16x4& hi, s16x4& lo) {
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const uint16_t h = f2bf(x[u]);
    hi[u] = (short)h;
    lo[u] = bfbits(x[u] - bf2f(h));
  }
}
}  // namespace

// With GATED the RMSNormGated epilogue (qwen3_5.rs:660-665) runs on the
// chunk's outputs: out[t, hv, :] = silu(z) * rms_norm(y, norm_w, norm_eps)
// over the Dv rows of the head, z read from the merged projection row
// (z = zrow + t * xs, columns hv*Dv ..); y is also stored when non-null.
template <int R, bool GATED>
__global__ __launch_bounds__(512) void prefill_chunk_kernel(
    float* __restrict__ state, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int num_slots, int Hk, int T,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ vc, const float* __restrict__ lgv,
    const uint16_t* __restrict__ betav, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ zrow, int64_t xs, const uint16_t* __restrict__ norm_w,
    float norm_eps, uint16_t* __restrict__ out, uint32_t* __restrict__ status) {
  constexpr int NT = 512;
  __shared__ ChunkSmem sm;
  const int hv = blockIdx.x, s = blockIdx.y;
  const int Hv = Hk * R, hk = hv / R;
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0 && hv == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  if (en <= st) return;
  // this lane's state row (accumulator column) and 4-row group
  float* gstate = state + ((size_t)slot * Hv + hv) * kTileElems + (size_t)(16 * w + (lane0 & 15)) * kDk +
                  4 * (lane0 >> 4);
  // RMSNormGated: the norm weight of this lane's output row, and its z column
  float nw = 0.f;
  const uint16_t* zcol = nullptr;
  if constexpr (GATED) {
    nw = bf2f(norm_w[16 * w + (lane0 & 15)]);
    zcol = zrow + (size_t)hv * kDv + 16 * w + (lane0 & 15);
  }

  // state accumulators: S^T tiles (dk block a, this wave's 16 state rows)
  f32x4 acc[8];
#pragma unroll
  for (int a = 0; a < 8; ++a)
    acc[a] = *reinterpret_cast<const f32x4*>(gstate + 16 * a);

  // chunk inputs in registers (prefetched one chunk ahead)
  uint4 kv[2], qv[2], vv[2];
  float pb = 0.f, pl = 0.f;
  auto load_inputs = [&](int c0) {
    const int n = min(kC, en - c0);
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + NT * u, i = e >> 4, c = (e & 15) * 8;
      kv[u] = make_uint4(0u, 0u, 0u, 0u);
      qv[u] = kv[u];
      vv[u] = kv[u];
      if (i < n) {
        const size_t off = ((size_t)(c0 + i) * Hk + hk) * kDk + c;
        kv[u] = *reinterpret_cast<const uint4*>(kn + off);
        qv[u] = *reinterpret_cast<const uint4*>(qn + off);
        vv[u] = *reinterpret_cast<const uint4*>(vc + ((size_t)(c0 + i) * Hv + hv) * kDv + c);
      }
    }
    pb = 0.f;
    pl = 0.f;
    if (w == 0 && lane0 < n) {
      pb = bf2f(betav[(size_t)(c0 + lane0) * Hv + hv]);
      pl = lgv[(size_t)(c0 + lane0) * Hv + hv];
    }
  };
  auto store_inputs = [&]() {
    // Opaque to the compiler until here, so it cannot unpack the prefetched
    // words (and wait for the loads) right after issuing them.
#pragma unroll
    for (int u = 0; u < 2; ++u)
      asm volatile("" : "+v"(kv[u].x), "+v"(kv[u].y), "+v"(kv[u].z), "+v"(kv[u].w),
                   "+v"(qv[u].x), "+v"(qv[u].y), "+v"(qv[u].z), "+v"(qv[u].w),
                   "+v"(vv[u].x), "+v"(vv[u].y), "+v"(vv[u].z), "+v"(vv[u].w));
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int e = tid + NT * u, i = e >> 4, c = (e & 15) * 8;
      *reinterpret_cast<uint4*>(&sm.K[i][c]) = kv[u];
      *reinterpret_cast<uint4*>(&sm.Q[i][c]) = qv[u];
      *reinterpret_cast<uint4*>(&sm.V[i][c]) = vv[u];
      const uint16_t* kb = reinterpret_cast<const uint16_t*>(&kv[u]);
#pragma unroll
      for (int x = 0; x < 8; ++x) sm.KT[c + x][kt_col(c + x, i)] = kb[x];
    }
    if (w == 0) {  // inclusive prefix sum of the log decay, in log2 units
      float gsum = pl * 1.4426950408889634f;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float t = __shfl_up(gsum, off, 64);
        if (lane0 >= off) gsum += t;
      }
      const float gC = __shfl(gsum, 63, 64);
      sm.beta[lane0] = pb;
      sm.G[lane0] = gsum;
      sm.eG[lane0] = __builtin_amdgcn_exp2f(gsum);
      sm.dec_end[lane0] = __builtin_amdgcn_exp2f(gC - gsum);
    }
  };

  load_inputs(st);
  for (int c0 = st; c0 < en; c0 += kC) {
    const int n = min(kC, en - c0);
    // Lane-derived LDS addresses are recomputed in every chunk (a few VALU
    // ops) instead of being held in registers across the loop.
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int lq = lane >> 4, lc = lane & 15;
    const int drow = 16 * w + lc;
    store_inputs();
    __syncthreads();
    if (c0 + kC < en) load_inputs(c0 + kC);

    // (b) waves 0-3: K K^T for token rows 16w.. -> -L (hi/lo) and its f32
    // diagonal block; waves 4-7: Q K^T for token rows 16(7-w).. -> P. Column
    // blocks above the row block are zero and skipped, so row block I has I+1
    // blocks; waves w and w+4 share a SIMD, which thus gets (w+1) + (4-w) = 5.
    {
      const int I = w < 4 ? w : 7 - w;
      const bool isq = w >= 4;
      const uint16_t* A = isq ? &sm.Q[0][0] : &sm.K[0][0];
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        if (J > I) continue;
        f32x4 c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
          c = mfma32(frag32(A, kLdK, 16 * I, 32 * ks, lane),
                     frag32(&sm.K[0][0], kLdK, 16 * J, 32 * ks, lane), c);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lq + r, j = 16 * J + lc;
          const float d = __builtin_amdgcn_exp2f(fminf(sm.G[i] - sm.G[j], 0.f));
          if (isq) {
            sm.P[i][j] = f2bf(j <= i ? c[r] * d : 0.f);
          } else {
            const float lv = j < i ? sm.beta[i] * c[r] * d : 0.f;
            const uint16_t nh = f2bf(-lv);
            sm.NLh[i][j] = nh;
            sm.NLl[i][j] = f2bf(-lv - bf2f(nh));
            if (J == I) sm.Ld[I][4 * lq + r][lc] = lv;
          }
        }
      }
    }
    // (c) waves 0-3: D_w = (I + L_ww)^-1 by forward substitution (lanes 0..15
    // = columns)
    if (w < 4 && lane < 16) {
      const int j = lane;
      float t[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        asm volatile("" ::: "memory");  // bound live ranges: one row of L at a time
        float a = i == j ? 1.f : 0.f;
#pragma unroll
        for (int k = 0; k < i; ++k) a -= sm.Ld[w][i][k] * t[k];
        t[i] = a;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint16_t h = f2bf(t[i]);
        sm.Dh[w][i][j] = h;
        sm.Dl[w][i][j] = f2bf(t[i] - bf2f(h));
      }
    }
    // (d) Y_I = K_I S^T and Z_I = Q_I S^T for this wave's 16 state rows; the
    // hi/lo split of the S^T accumulator tiles is the B operand
    f32x4 yk[4], zq[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      yk[I] = f32x4{0.f, 0.f, 0.f, 0.f};
      zq[I] = yk[I];
    }
#pragma unroll
    for (int a = 0; a < 8; ++a) {
      asm volatile("" ::: "memory");  // bound live ranges: one dk block at a time
      s16x4 sh, sl;
      split4(acc[a], sh, sl);
      const bf16x8 bs = cat(sh, sl);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const s16x4 ak = frag16(&sm.K[0][0], kLdK, 16 * I, 16 * a, lane);
        const s16x4 aq = frag16(&sm.Q[0][0], kLdK, 16 * I, 16 * a, lane);
        yk[I] = mfma32(cat(ak, ak), bs, yk[I]);
        zq[I] = mfma32(cat(aq, aq), bs, zq[I]);
      }
    }
    __syncthreads();

    // (e, f) R_I, then V'_I = D_I (R_I - sum_{j<I} L_Ij V'_j)
    s16x4 vph[4], vpl[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 x;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lq + r;
        x[r] = sm.beta[i] * (bf2f(sm.V[i][drow]) - sm.eG[i] * yk[I][r]);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j >= I) continue;
        const s16x4 lh = frag16(&sm.NLh[0][0], kLdT, 16 * I, 16 * j, lane);
        const s16x4 ll = frag16(&sm.NLl[0][0], kLdT, 16 * I, 16 * j, lane);
        x = mfma32(cat(lh, ll), cat(vph[j], vph[j]), x);  // lh.vph + ll.vph
        x = mfma32(cat(lh, kZero4), cat(vpl[j], vpl[j]), x);  // lh.vpl
      }
      s16x4 xh, xl;
      split4(x, xh, xl);
      const s16x4 dh = frag16(&sm.Dh[I][0][0], kLdD, 0, 0, lane);
      const s16x4 dl = frag16(&sm.Dl[I][0][0], kLdD, 0, 0, lane);
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      v = mfma32(cat(dh, dl), cat(xh, xh), v);      // dh.xh + dl.xh
      v = mfma32(cat(dh, kZero4), cat(xl, xl), v);  // dh.xl
      split4(v, vph[I], vpl[I]);
    }
    // (g) O_I = exp(G) * Z_I + sum_{j<=I} P_Ij V'_j
    float yo[4][4];      // GATED: y of tokens 16I + 4lq + r, row drow (bf16 values)
    uint16_t zv[4][4];   // GATED: z of the same outputs
    if constexpr (GATED) {  // issued first, consumed after the y^2 sums
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          zv[I][r] = zcol[(size_t)min(c0 + 16 * I + 4 * lq + r, en - 1) * xs];
    }
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 o;
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = zq[I][r] * sm.eG[16 * I + 4 * lq + r];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j > I) continue;
        const s16x4 ph = frag16(&sm.P[0][0], kLdT, 16 * I, 16 * j, lane);
        o = mfma32(cat(ph, ph), cat(vph[j], vpl[j]), o);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * I + 4 * lq + r;
        if constexpr (GATED) {
          yo[I][r] = rbf(o[r]);
          // sum of y^2 over this wave's 16 rows (the 16 lanes of the DPP row)
          const float ss = sum16(yo[I][r] * yo[I][r]);
          if (lc == 0) sm.ysq[i][w] = ss;
        }
        if (y != nullptr && i < n) y[((size_t)(c0 + i) * Hv + hv) * kDv + drow] = f2bf(o[r]);
      }
    }
    if constexpr (GATED) {  // RMSNormGated over the Dv = 128 rows of each token
      __syncthreads();
#pragma unroll
      for (int I = 0; I < 4; ++I)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * I + 4 * lq + r;
          const f32x4 p0 = *reinterpret_cast<const f32x4*>(&sm.ysq[i][0]);
          const f32x4 p1 = *reinterpret_cast<const f32x4*>(&sm.ysq[i][4]);
          const float tot = ((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p1[0] + p1[1]) + (p1[2] + p1[3]));
          const float rn = 1.0f / sqrtf(tot / (float)kDv + norm_eps);
          const float normed = rbf(nw * rbf(yo[I][r] * rn));
          if (i < n)
            out[((size_t)(c0 + i) * Hv + hv) * kDv + drow] = f2bf(silu_bf16(bf2f(zv[I][r])) * normed);
        }
    }
    // (h) S^T <- exp(G_C) S^T + K^T (exp(G_C - G) * V')
    const float eC = sm.eG[kC - 1];
#pragma unroll
    for (int a = 0; a < 8; ++a) acc[a] *= eC;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      asm volatile("" ::: "memory");  // bound live ranges: one token block at a time
      f32x4 vt;
#pragma unroll
      for (int r = 0; r < 4; ++r)
        vt[r] = (bf2f((uint16_t)vph[j][r]) + bf2f((uint16_t)vpl[j][r])) *
                sm.dec_end[16 * j + 4 * lq + r];
      s16x4 th, tl;
      split4(vt, th, tl);
      const bf16x8 bt = cat(th, tl);
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        const s16x4 kt = frag16_kt(sm.KT, 16 * a, 16 * j, lane);
        acc[a] = mfma32(cat(kt, kt), bt, acc[a]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 8; ++a)
    *reinterpret_cast<f32x4*>(gstate + 16 * a) = acc[a];
}

size_t prefill_workspace_bytes(int R, int Hk, int total_tokens) {
  return carve(nullptr, R, Hk, total_tokens, nullptr);
}

// ---------------------------------------------------- no-allocation scratch --
// Workspace of gdn_prefill_varlen_noalloc: one fixed array per device, in
// place of the pool's grown workspace. Every call on a device shares it and
// finds the previous call's contents (the prefill writes every workspace byte
// it reads, so nothing needs clearing); calls that overlap on one device race.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

size_t noalloc_scratch_bytes() { return kNoAllocScratchBytes; }

// The device address of `scratch` on the current device, looked up once per
// device (the host-side name of the array is not a device address).
hipError_t noalloc_scratch(void** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static void* ptrs[kMaxDevices] = {};
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(mu);
  if (!ptrs[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    ptrs[dev] = p;
  }
  *out = ptrs[dev];
  return hipSuccess;
}

template <int R>
static hipError_t launch_prefill_r(const PrefillArgs& a) {
  const int Hv = a.Hk * R;
  const int D = 2 * a.Hk * kDk + Hv * kDv;
  Workspace ws;
  carve(a.workspace, R, a.Hk, a.total_tokens, &ws);
  if (a.total_tokens > 0) {
    hipLaunchKernelGGL(prefill_qkv_kernel<R>, dim3(2 * a.Hk + Hv, (a.total_tokens + kTT - 1) / kTT),
                       dim3(256), 0, a.stream, a.conv, a.slot_ids, a.cu_seqlens, a.nseq,
                       a.num_slots, a.Hk, a.total_tokens, a.mixed, a.xstride, a.conv_w, a.ab,
                       a.ab_stride, a.A_log,
                       a.dt_bias, ws.qn, ws.kn, ws.vc, ws.beta, ws.lg);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(prefill_conv_state_kernel, dim3(a.nseq, (D + 255) / 256), dim3(256), 0,
                     a.stream, a.conv, a.slot_ids, a.cu_seqlens, a.nseq, a.num_slots, D,
                     a.total_tokens, a.mixed, a.xstride, a.status);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.out)
    hipLaunchKernelGGL((prefill_chunk_kernel<R, true>), dim3(Hv, a.nseq), dim3(512), 0,
                       a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk,
                       a.total_tokens, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, a.y, a.mixed + D,
                       a.xstride, a.norm_w, a.norm_eps, a.out, a.status);
  else
    hipLaunchKernelGGL((prefill_chunk_kernel<R, false>), dim3(Hv, a.nseq), dim3(512), 0,
                       a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk,
                       a.total_tokens, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, a.y, nullptr,
                       a.xstride, nullptr, 0.0f, nullptr, a.status);
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
