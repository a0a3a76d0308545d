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

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <type_traits>

#include "gdn_common.h"

namespace gdn {

namespace {

constexpr float kQNormW = 0.0078125f;
constexpr float kKNormW = 0.08837890625f;
constexpr float kNormEps = 1e-6f;
constexpr int kTT = 64;  // tokens per qkv_kernel work-group
// The split path is taken for prompts of at least kSplitMinTokens tokens on
// average and calls of at most kSplitMaxTokens tokens (its records take 272
// bytes per token and value head).
constexpr int kSplitMinTokens = 1024;
constexpr int kSplitMaxTokens = 1 << 18;
constexpr int kRecStride = 17408;  // bytes per chunk record (kRecBytes)

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

struct Workspace {
  uint16_t* qn;
  uint16_t* kn;
  uint16_t* vc;
  uint16_t* beta;
  float* lg;
  uint16_t* rec;  // split path: chunk records [floor(T/64) + nseq][Hv] of 17,408 bytes
  uint16_t* y;    // split path with the gated epilogue and no y from the caller: [T, Hv, Dv]
};

size_t carve(void* base, int R, int Hk, int T, int nseq, int waves, bool y_scratch, Workspace* w) {
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
  ws.rec = nullptr;
  ws.y = nullptr;
  if (waves < 8) {
    ws.rec = static_cast<uint16_t*>(take((size_t)(T / 64 + nseq) * Hv * kRecStride));
    if (y_scratch) ws.y = static_cast<uint16_t*>(take((size_t)T * Hv * kDv * 2));
  }
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
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

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
// of one token. grid (2Hk+Hv, tiles), block 256: token tiles tile0 ..
// tile0 + tiles - 1 (all ceil(T/64) of them, or one segment of a pipelined
// call).
template <int R>
__global__ __launch_bounds__(256) void prefill_qkv_kernel(
    const uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int nseq, int num_slots, int Hk, int T, int tile0,
    const uint16_t* __restrict__ x, int64_t xs, const uint16_t* __restrict__ conv_w,
    const uint16_t* __restrict__ ab, int64_t abs_, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, uint16_t* __restrict__ qn, uint16_t* __restrict__ kn,
    uint16_t* __restrict__ vc, uint16_t* __restrict__ beta, float* __restrict__ lg) {
  constexpr int KH = kConvK - 1;
  __shared__ uint4 tile[kTT + KH][16];
  __shared__ int tok_st[kTT];    // first token of the token's sequence (clamped <= t)
  __shared__ int tok_slot[kTT];  // slot of that sequence, -1 if invalid
  const int head = blockIdx.x, t0 = (blockIdx.y + tile0) * kTT;
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
      // the 16 lanes of the token: DPP adds in xor 1, 2, 4, 8 partner order
      // (the bits of an xor-shuffle butterfly, without the LDS crossbar)
      ss = sum16(ss);
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
    // streamed past the caches: the chunk kernel reads the 2 GB of outputs
    // back from HBM either way
    if (t < T) __builtin_nontemporal_store(u32x4{o[0], o[1], o[2], o[3]}, reinterpret_cast<u32x4*>(dst) + l);
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

// 3. Chunked (WY form) recurrence. With G the cumulative log decay inside a
// chunk of kC = 64 tokens and S ([Dv, Dk]) the state at the chunk start:
//   L_ij = beta_i (k_i.k_j) exp(G_i - G_j)   (j < i)
//   P_ij = (q_i.k_j) exp(G_i - G_j)          (j <= i)
//   R    = beta * (V - exp(G) * (K S^T))      per token row
//   (I + L) V' = R                            (block forward substitution)
//   O    = exp(G) * (Q S^T) + P V'
//   S^T <- exp(G_C) S^T + K^T (exp(G_C - G) * V')
// which equals the token-by-token recurrence of metal_gdn.rs:37-62.
//
// Work split. One work-group of 8 waves per (sequence, value head), each wave
// owning 16 of the 128 state rows (the rows of S evolve independently). The
// group forms the chunk's state-independent matrices itself: each of four
// waves takes one diagonal 16x16 block of L and inverts it, D_I = (I +
// L_II)^-1, while the waves share the off-diagonal blocks of L and the blocks
// of P. Every wave then works on its own 16 state rows, held in MFMA
// accumulators across chunks. A chunk needs three work-group barriers: inputs
// staged, matrices formed, chunk done.
//
// Operand layouts of v_mfma_f32_16x16x32_bf16 (lane l, q = l/16, c = l%16):
// an A operand holds row c, k slots 8q..8q+7; a B operand column c, the same k
// slots; the accumulator holds row 4q + r, column c in register r. Two 16-row
// accumulator tiles side by side, cat(X, X'), form an operand whose k slots
// 8q..8q+3 are rows 4q..4q+3 of X and 8q+4..8q+7 the same rows of X'; the
// other operand reads its k values in that "pair order". Q and P rows are
// stored in pair order so that such an operand is one 16-byte LDS read. K is
// stored in natural dk order with its 8-byte segments XOR-swizzled per row:
// the pair-order reads (two segments) and the transposing reads of the state
// update (ds_read_b64_tr_b16, four rows of one column block) both spread over
// the LDS banks.
//
// Precision: k and q are bf16, exact MFMA operands. f32 operands of the
// products that feed the state (S in K S^T, -L, D, the solve's right-hand
// sides, V') are split into bf16 hi + lo (~16 mantissa bits); the products
// that only reach the bf16 outputs (Q S^T, P V') use hi alone. Padded rows of
// a partial chunk have k = q = beta = 0, v = 0 and log decay 0, so they change
// nothing.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kC = 64;
// LDS on gfx950 (measured with SQ_LDS_BANK_CONFLICT on single access
// patterns): reads are served 256 bytes per cycle from 64 banks of 4 bytes,
// a pass being 64 lanes of a 4-byte read, 32 lanes of an 8-byte read, and
// lanes 0-7 with 16-23 (or 8-15 with 24-31) of a 16-byte read; writes are
// served 128 bytes per cycle from 32 banks, a pass being 32 lanes of a 4-byte
// write, 16 of an 8-byte and 8 of a 16-byte write. Lanes of one pass that hit
// one bank at different addresses serialize.
//
// Row strides: the 16-byte operand reads below (lane (q, c): row c, 16-byte
// column group q) are conflict-free when the stride is 8 mod 16 dwords. The
// writes of L and P blocks (lane c: row c) then meet rows c and c + 4 (mod 8)
// in one bank group; their 16-byte column groups are XORed with bit 2 of the
// row (gsw), which the reads undo.
constexpr int kLdQ = kDk + 16;     // Q rows in pair order (288 B = 72 dwords)
constexpr int kLdP = kC + 16;      // P rows in pair order (160 B = 40 dwords)
constexpr int kLdN = 2 * kC + 16;  // -L rows: 16 groups of (4 hi, 4 lo) (288 B)
constexpr int kLdD = 48;           // D_I rows: 4 groups of (4 hi, 4 lo) (96 B = 24 dwords)
constexpr int kLdDB = 16 * kLdD + 32;  // D_I blocks: the 4 blocks start 16 banks apart
constexpr int kLdL = 20;           // rows of the diagonal blocks of L, f32 (80 B)
constexpr int kLdLB = 16 * kLdL + 8;
constexpr int kKBlk = 16 * kDk + 64;   // K: 16-row blocks, 64 elements of padding between

// 16-byte column group g of row `row` of NL or P is stored at group g ^ gsw(row).
__device__ __forceinline__ int gsw(int row) { return (row >> 2) & 1; }
// Input unit e (0..1023) of q: chunk row qrow(e), 16-byte unit qunit(e) of
// the row (lanes 0-7 units 0-7 of an even row, lanes 8-15 the same of the
// next row, lanes 16-31 units 8-15 of the two rows).
__device__ __forceinline__ int qrow(int e) { return 2 * (e >> 5) + ((e >> 3) & 1); }
__device__ __forceinline__ int qunit(int e) { return (e & 7) + 8 * ((e >> 4) & 1); }

struct __attribute__((aligned(16))) ChunkSmem {
  static constexpr int kNLRow0 = 16;  // block row 0 of -L has no block left of the diagonal
  static constexpr int kLdV = kLdQ;   // row strides of V and Y
  static constexpr int kLdY = kDv + 4;
  uint16_t K[4 * kKBlk];       // k, natural dk order, segments swizzled (kseg)
  uint16_t Q[kC][kLdQ];        // q, dk in pair order: 32b + 16h + 4m + u at 32b + 8m + 4h + u
  uint16_t P[kC][kLdP];        // P, token columns in pair order; blocks above the diagonal stay 0
  uint16_t NL[kC - 16][kLdN];  // -L rows 16..63, hi/lo interleaved per 4 columns
  uint16_t D[4 * kLdDB];       // D_I, rows of kLdD, hi/lo interleaved per 4 columns
  float Ld[4 * kLdLB];         // diagonal blocks of L (f32): row i, column 4m + p at 4p + m
  float beta[kC], G[kC], eG[kC], dec[kC];  // G: cumulative log2 decay
  uint16_t V[kC][kLdV];        // v rows (row stride 288 B: the transposing reads of 8
                               // consecutive rows x 32 bytes hit distinct banks)
  uint16_t Y[kC][kLdY];        // the chunk's outputs y (bf16), written out as whole rows; the
                               // 66-dword stride puts the 16 rows of an 8-byte write pass and
                               // the 2 rows of an 8-byte read pass in distinct banks
  float ysq[kC][8];            // gated epilogue: per token, each wave's sum of y^2
};

// LDS of the split path's chunk kernel (W waves, 16W state rows): what the
// chain needs, about 77 KB at W = 2, so that a form-kernel group fits beside
// it on a CU. Block row 0 of -L has no block left of the diagonal, so -L
// starts at row 16; v and y hold the group's 16W columns (relative to its
// first state row). Row strides: v 32W + 32 bytes, so the transposing reads
// of 8 consecutive rows x 32 bytes still hit distinct banks; y 32W + 8 bytes,
// so the 16 rows of an 8-byte write pass of the O tiles do. No diagonal-block
// scratch, no G, no gated-epilogue sums.
template <int W>
struct __attribute__((aligned(16))) SplitSmem {
  static constexpr int kNLRow0 = 16;
  static constexpr int kLdV = 16 * W + 16;
  static constexpr int kLdY = 16 * W + 4;
  uint16_t K[4 * kKBlk];
  uint16_t Q[kC][kLdQ];
  uint16_t P[kC][kLdP];
  uint16_t NL[kC - 16][kLdN];
  uint16_t D[4 * kLdDB];
  float beta[kC], eG[kC], dec[kC];
  uint16_t V[kC][kLdV];
  uint16_t Y[kC][kLdY];
};

// Row `row` of -L (row >= S::kNLRow0)
template <class S>
__device__ __forceinline__ uint16_t* nl_row(S& sm, int row) { return sm.NL[row - S::kNLRow0]; }
template <class S>
__device__ __forceinline__ const uint16_t* nl_row(const S& sm, int row) { return sm.NL[row - S::kNLRow0]; }

// DPP move of a float (lanes without a source read 0)
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
}
__device__ __forceinline__ f32x4 mfma32(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ __forceinline__ bf16x8 cat(s16x4 a, s16x4 b) {
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7));
}
__device__ __forceinline__ s16x4 lds4(const uint16_t* p) {
  return *static_cast<const s16x4*>(__builtin_assume_aligned(p, 8));
}
__device__ __forceinline__ bf16x8 lds8(const uint16_t* p) {
  return *static_cast<const bf16x8*>(__builtin_assume_aligned(p, 16));
}
constexpr s16x4 kZero4 = {0, 0, 0, 0};

// Element offset of the natural 4-dk segment s (dk 4s..4s+3) of K row `row`.
// LDS has 64 banks of 4 bytes and serves an 8-byte access 32 lanes at a time.
// Within a block of 16 rows the swizzle g(r) = (r & 7) << 2 | ((r >> 3) & 1)
// << 1 (r = row % 16) puts the 32 segments of such a pass in 32 distinct bank
// pairs for both access forms: a pair-order read (16 consecutive rows,
// segments differing in bit 0; bits 1-4 of g run through 0..15) and a
// transposing read (8 consecutive rows x 4 consecutive segments; bits 2-4 of g
// run through 0..7). The 16-row blocks are kKBlk = 16*128 + 64 elements apart:
// rows 16 apart are then 4224 bytes apart, a distance no ds_read2 form encodes,
// so the compiler cannot fuse two rows' reads into one ds_read2st64_b64 whose
// two addresses would share a bank (measured: 16 conflict cycles per pair).
// For a fixed lane the offset is a lane constant XOR a compile-time constant
// plus a compile-time block offset, so an operand read costs one VALU op.
__device__ __forceinline__ int kseg(int row, int s) {
  const int r = row & 15;
  return (row >> 4) * kKBlk + r * kDk + 4 * (s ^ (((r & 7) << 2) | (((r >> 3) & 1) << 1)));
}
// K operand reads from per-lane constants: with kf = kseg(c, q), the pair-order
// operand of row 16X + c, dk block b (32 values) reads segments 8b + q and
// 8b + 4 + q at X*kKBlk + (kf ^ (32b + 16h)), h = 0, 1 (the XORed bits and the
// row bits of kseg are disjoint).
__device__ __forceinline__ bf16x8 kfrag(const uint16_t* K, int kf, int X, int b) {
  return cat(lds4(K + X * kKBlk + (kf ^ (32 * b))), lds4(K + X * kKBlk + (kf ^ (32 * b + 16))));
}
// K^T operand rows for the state update: lane (q, c) receives
// K[16 blk + 4q + u][16a + c], u = 0..3. ds_read_b64_tr_b16 hands lane j of a
// 16-lane group element j of the 4 x 16 block whose row u the lanes 4u..4u+3
// read, 4 elements each; lane 4u + s reads row 4q + u, segment 4a + s at
// blk*kKBlk + (kt ^ 16a) with kt = kseg(4q + (i >> 2), i & 3), i = lane % 16.
typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
__device__ __forceinline__ s16x4 ktr(const uint16_t* K, int kt, int blk, int a) {
  lds_bf16x4* p = (lds_bf16x4*)(K + blk * kKBlk + (kt ^ (16 * a)));
  return __builtin_bit_cast(s16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(p));
}

// v operand of the solve, a transposing read like ktr: lane (q, c) passes
// row 16I + 4q + (c >> 2) and column dv0 + 4(c & 3) and receives
// V[16I + 4q + u][dv0 + c], u = 0..3.
template <class S>
__device__ __forceinline__ s16x4 vtr(const S& sm, int row, int col) {
  lds_bf16x4* p = (lds_bf16x4*)&sm.V[row][col];
  return __builtin_bit_cast(s16x4, __builtin_amdgcn_ds_read_tr16_b64_v4bf16(p));
}

// f32 -> bf16 hi + lo (hi + lo carries ~16 mantissa bits). The arithmetic
// shared by the fused and the split path is written so that the compiler
// cannot fuse a product with a following add in one kernel and not in the
// other (it decides per basic block): explicit fmaf where a fused operation is
// meant, contraction off where a product is rounded on its own. Both paths
// then give the same bits.
__device__ __forceinline__ void split4(const f32x4& x, s16x4& hi, s16x4& lo) {
#pragma clang fp contract(off)
  const uint32_t h0 = f2bf2(x[0], x[1]), h1 = f2bf2(x[2], x[3]);
  const uint32_t l0 = f2bf2(x[0] - bf_lo(h0), x[1] - bf_hi(h0));
  const uint32_t l1 = f2bf2(x[2] - bf_lo(h1), x[3] - bf_hi(h1));
  hi = __builtin_bit_cast(s16x4, (uint2){h0, h1});
  lo = __builtin_bit_cast(s16x4, (uint2){l0, l1});
}
__device__ __forceinline__ s16x4 hi4(const f32x4& x) {
  return __builtin_bit_cast(s16x4, (uint2){f2bf2(x[0], x[1]), f2bf2(x[2], x[3])});
}

// L block (I, J), J <= I: an off-diagonal block as -L hi/lo into NL (row
// 16I+c, columns 16J+4q..+3), a diagonal block into Ld in f32.
template <class S>
__device__ __forceinline__ void put_l(S& sm, const f32x4& t, int I, int J, int q, int c) {
  const int i = 16 * I + c;
  const float Gi = sm.G[i], bi = sm.beta[i];
  const f32x4 Gj = *reinterpret_cast<const f32x4*>(&sm.G[16 * J + 4 * q]);
  f32x4 lv;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = bi * t[r] * __builtin_amdgcn_exp2f(fminf(Gi - Gj[r], 0.f));
    lv[r] = (J < I || 4 * q + r < c) ? v : 0.f;
  }
  if (J == I) {
    // row c of the block, column 4q + r at place 4r + q (the inversion's lane
    // p reads columns p, p+4, p+8, p+12 as one 16-byte group)
#pragma unroll
    for (int r = 0; r < 4; ++r) sm.Ld[I * kLdLB + c * kLdL + 4 * r + q] = lv[r];
  } else {
    s16x4 h, l;
    split4(-lv, h, l);
    *reinterpret_cast<bf16x8*>(nl_row(sm, i) + 32 * J + 8 * (q ^ gsw(c))) = cat(h, l);
  }
}
// P block (I, J), J <= I: row 16I+c, columns 16J+4q..+3 at their pair-order place.
template <class S>
__device__ __forceinline__ void put_p(S& sm, const f32x4& t, int I, int J, int q, int c) {
  const int i = 16 * I + c;
  const float Gi = sm.G[i];
  const f32x4 Gj = *reinterpret_cast<const f32x4*>(&sm.G[16 * J + 4 * q]);
  f32x4 pv;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const float v = t[r] * __builtin_amdgcn_exp2f(fminf(Gi - Gj[r], 0.f));
    pv[r] = (J < I || 4 * q + r <= c) ? v : 0.f;
  }
  *static_cast<s16x4*>(__builtin_assume_aligned(&sm.P[i][32 * (J >> 1) + 8 * (q ^ gsw(c)) + 4 * (J & 1)], 8)) =
      hi4(pv);
}

// The operand fragments of one 16-row block for the four 32-wide dk blocks:
// K rows (kfrags) or Q rows (qfrags) 16X + c, 16-byte column group q.
struct Frag {
  bf16x8 f[4];
};
template <class S>
__device__ __forceinline__ Frag kfrags(const S& sm, int kf, int X) {
  Frag r;
#pragma unroll
  for (int b = 0; b < 4; ++b) r.f[b] = kfrag(sm.K, kf, X, b);
  return r;
}
template <class S>
__device__ __forceinline__ Frag qfrags(const S& sm, int X, int q, int c) {
  Frag r;
#pragma unroll
  for (int b = 0; b < 4; ++b) r.f[b] = lds8(&sm.Q[16 * X + c][32 * b + 8 * q]);
  return r;
}
// Tiles of the chunk's matrices, as accumulators holding row 4q + r, column c:
// tile(K_J, K_I) = (K K^T)[16I+c][16J+4q+r] and tile(K_J, Q_I) =
// (Q K^T)[16I+c][16J+4q+r]: lane c owns row 16I+c of L or P.
__device__ __forceinline__ f32x4 tile(const Frag& colJ, const Frag& rowI) {
  f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int b = 0; b < 4; ++b) t = mfma32(colJ.f[b], rowI.f[b], t);
  return t;
}

// The 16 blocks besides the diagonal blocks of L (6 off-diagonal blocks of L,
// the 10 blocks of P (I, J), J <= I), four per wave for waves 4-7, grouped so
// that a wave's four tiles share operand blocks (4-5 blocks of 16 rows).
// Each wave's code is straight-line: all its LDS operand reads are in flight
// together instead of one tile's reads at a time.
template <class S>
__device__ __forceinline__ void other_blocks(S& sm, int w, int kf, int q, int c) {
  if (w == 4) {
    const Frag k0 = kfrags(sm, kf, 0), k1 = kfrags(sm, kf, 1), k2 = kfrags(sm, kf, 2),
               k3 = kfrags(sm, kf, 3), q3 = qfrags(sm, 3, q, c);
    put_l(sm, tile(k0, k3), 3, 0, q, c);
    put_l(sm, tile(k1, k3), 3, 1, q, c);
    put_l(sm, tile(k2, k3), 3, 2, q, c);
    put_p(sm, tile(k3, q3), 3, 3, q, c);
  } else if (w == 5) {
    const Frag k0 = kfrags(sm, kf, 0), k1 = kfrags(sm, kf, 1), k2 = kfrags(sm, kf, 2),
               q3 = qfrags(sm, 3, q, c);
    put_p(sm, tile(k0, q3), 3, 0, q, c);
    put_p(sm, tile(k1, q3), 3, 1, q, c);
    put_p(sm, tile(k2, q3), 3, 2, q, c);
    put_l(sm, tile(k0, k2), 2, 0, q, c);
  } else if (w == 6) {
    const Frag k0 = kfrags(sm, kf, 0), k1 = kfrags(sm, kf, 1), k2 = kfrags(sm, kf, 2),
               q2 = qfrags(sm, 2, q, c);
    put_p(sm, tile(k0, q2), 2, 0, q, c);
    put_p(sm, tile(k1, q2), 2, 1, q, c);
    put_p(sm, tile(k2, q2), 2, 2, q, c);
    put_l(sm, tile(k1, k2), 2, 1, q, c);
  } else if (w == 7) {
    const Frag k0 = kfrags(sm, kf, 0), k1 = kfrags(sm, kf, 1), q0 = qfrags(sm, 0, q, c),
               q1 = qfrags(sm, 1, q, c);
    put_p(sm, tile(k0, q0), 0, 0, q, c);
    put_p(sm, tile(k0, q1), 1, 0, q, c);
    put_p(sm, tile(k1, q1), 1, 1, q, c);
    put_l(sm, tile(k0, k1), 1, 0, q, c);
  }
}

// Wave 0, lane l = token l of the chunk (raw bf16 beta b, log decay lg):
// beta, the cumulative decay G in log2 units (an inclusive prefix sum over the
// 64 lanes on DPP: shifts within each 16-lane row, then row 0's and row 2's
// totals into rows 1 and 3 (row_bcast:15), then the first half's total into
// rows 2 and 3 (row_bcast:31)), exp2(G) and the decay to the chunk's end.
template <class S>
__device__ __forceinline__ void form_gates(S& sm, uint16_t b, float lg, int lane) {
#pragma clang fp contract(off)
  float gsum = lg * 1.4426950408889634f;
  gsum += dpp_f<0x111, 0xF>(gsum);  // row_shr:1
  gsum += dpp_f<0x112, 0xF>(gsum);  // row_shr:2
  gsum += dpp_f<0x114, 0xF>(gsum);  // row_shr:4
  gsum += dpp_f<0x118, 0xF>(gsum);  // row_shr:8
  gsum += dpp_f<0x142, 0xA>(gsum);  // row_bcast:15
  gsum += dpp_f<0x143, 0xC>(gsum);  // row_bcast:31
  const float gC = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(gsum), 63));
  sm.beta[lane] = bf2f(b);
  sm.G[lane] = gsum;
  sm.eG[lane] = __builtin_amdgcn_exp2f(gsum);
  sm.dec[lane] = __builtin_amdgcn_exp2f(gC - gsum);
}

// Wave I (0..3): diagonal block I of L and its inverse D_I = (I + L_II)^-1 by
// forward substitution with four lanes per column: lane (j = l/4, p = l%4)
// sums the terms k = p (mod 4) of each row and two DPP adds close the sum
// over its quad, so a row costs a handful of dependent VALU ops.
template <class S>
__device__ __forceinline__ void invert_diag(S& sm, int I, int kf, int q, int c, int lane) {
  const Frag kI = kfrags(sm, kf, I);
  put_l(sm, tile(kI, kI), I, I, q, c);
  // this wave's own Ld writes, read back by other lanes of the wave
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
  const int j = lane >> 2, pp = lane & 3;
  const float* Lb = &sm.Ld[I * kLdLB + 4 * pp];
  float tv[4] = {pp == 0 && j == 0 ? 1.f : 0.f, 0.f, 0.f, 0.f};  // t_{4m+p} of column j
  f32x4 row = *reinterpret_cast<const f32x4*>(&Lb[kLdL]);
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const f32x4 cur = row;
    if (i + 1 < 16) row = *reinterpret_cast<const f32x4*>(&Lb[(i + 1) * kLdL]);
    float part = 0.f;
#pragma unroll
    for (int m = 0; m <= (i - 1) >> 2; ++m) part = fmaf(cur[m], tv[m], part);
    part += dpp_f<0xB1, 0xF>(part);  // quad_perm xor 1
    part += dpp_f<0x4E, 0xF>(part);  // quad_perm xor 2
    const float ti = (i == j ? 1.f : 0.f) - part;
    if (pp == (i & 3)) tv[i >> 2] = ti;
  }
  // rows 4m + p of column j, hi and lo
  uint16_t* Dp = &sm.D[I * kLdDB + 8 * (j >> 2) + (j & 3)];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint16_t h = f2bf(tv[m]);
    Dp[(4 * m + pp) * kLdD] = h;
    Dp[(4 * m + pp) * kLdD + 4] = f2bf(tv[m] - bf2f(h));
  }
}

// Record of one (chunk, value head) for the split path: the operands of the
// chunk's state products that do not depend on the state, in 16-byte units u
// (rec_slot gives each unit's place in the LDS layouts above):
//   [0, 384)      -L, rows 16..63: row 16I + i (I = 1..3) holds the 4I column
//                 groups of its blocks left of the diagonal (hi/lo per 4 columns)
//   [384, 640)    D, block I, row i: 4 groups
//   [640, 1024)   P, rows 0..31 groups 0-3, rows 32..63 groups 0-7 (pair order;
//                 the halves above the diagonal are 0)
//   [1024, 1072)  beta, exp2(G), exp2(G_C - G): 16 units each (f32)
constexpr int kRecUnits = 1072;
constexpr int kRecBytes = kRecStride;  // record stride (256-byte aligned)
static_assert(kRecBytes >= kRecUnits * 16 && kRecBytes % 256 == 0, "record stride");
template <class S>
__device__ __forceinline__ void* rec_slot(S& sm, int u) {
  if (u < 384) {
    int row, g;
    if (u < 64) {
      row = 16 + (u >> 2);
      g = u & 3;
    } else if (u < 192) {
      row = 32 + ((u - 64) >> 3);
      g = (u - 64) & 7;
    } else {
      const int off = u - 192, r = off / 12;
      row = 48 + r;
      g = off - 12 * r;
    }
    return nl_row(sm, row) + 8 * (g ^ gsw(row));
  }
  if (u < 640) {
    const int v = u - 384;
    return &sm.D[(v >> 6) * kLdDB + ((v >> 2) & 15) * kLdD + 8 * (v & 3)];
  }
  if (u < 1024) {
    const int v = u - 640;
    const int row = v < 128 ? v >> 2 : 32 + ((v - 128) >> 3);
    const int g = v < 128 ? v & 3 : (v - 128) & 7;
    return &sm.P[row][8 * (g ^ gsw(row))];
  }
  const int v = u - 1024, k = 4 * (v & 15);
  return v < 16 ? &sm.beta[k] : v < 32 ? &sm.eG[k] : &sm.dec[k];
}

// Sum of squares of 4 bf16 outputs, and the RMSNormGated output of 8 rows
// (silu(z) * bf16(w * bf16(y * rn))), shared by the chunk kernel's epilogue
// and the split path's separate epilogue so that both give the same bits.
__device__ __forceinline__ float sumsq4(float a, float b, float c, float d) {
  return fmaf(b, b, a * a) + fmaf(d, d, c * c);
}
__device__ __forceinline__ float rms_scale(float tot, float eps) {
  return 1.0f / sqrtf(tot / (float)kDv + eps);
}
__device__ __forceinline__ u32x4 norm_gate8(const u32x4& yv, const u32x4& zv, const u32x4& nw, float rn) {
  u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float o0 = silu_bf16(bf_lo(zv[e])) * rbf(bf_lo(nw[e]) * rbf(bf_lo(yv[e]) * rn));
    const float o1 = silu_bf16(bf_hi(zv[e])) * rbf(bf_hi(nw[e]) * rbf(bf_hi(yv[e]) * rn));
    o[e] = f2bf2(o0, o1);
  }
  return o;
}
}  // namespace

// Record slot of chunk k of sequence s (first token st): floor(st/64) + s + k.
// Over a call the slots are distinct and below floor(T/64) + nseq: sequence s
// has at most floor(st_{s+1}/64) - floor(st_s/64) + 1 chunks.
inline int rec_slots(int T, int nseq) { return T / kC + nseq; }

// With GATED the RMSNormGated epilogue (qwen3_5.rs:660-665) runs on the
// chunk's outputs: out[t, hv, :] = silu(z) * rms_norm(y, norm_w, norm_eps)
// over the Dv rows of the head, z read from the merged projection row
// (z = zrow + t * xs, columns hv*Dv ..); y is also stored when non-null.
//
// One work-group of 8 waves per (sequence, value head): the chunks of a
// sequence are a serial chain, so the time per chunk of one group sets the
// kernel time; splitting a head's rows over more, smaller groups lengthens it
// (measured for one 16,384-token prompt: 1.49 ms with 32 groups of 8 waves,
// 1.79 ms with 64 of 4, 2.26 ms with 128 of 2). The chunk's outputs go
// through LDS and leave as whole 256-byte rows.
//
// Split path (W = 2 or 4): the chunk's blocks of L and P, the inverses D_I
// and the gates come from the records of prefill_form_kernel, and each
// (sequence, value head) has 8/W groups of W waves, each group 16W state
// rows; without the block formation the groups need no barrier between
// the products and the solve. The split path has no GATED epilogue (the
// norm runs over all 128 rows of a head; prefill_norm_gate_kernel does it).
//
// 1D grid of Hv * nseq * (8/W) groups. Work-groups are dealt to the 8 XCDs
// round-robin; the R * 8/W groups that read one key head's k and q are
// numbered 8 apart, so they run on one XCD and fetch those rows once.
//
// A launch runs the chunks whose last token + 1 lies in (plo, phi] (0 and T:
// all of them), from the state in the slot and back into it: a pipelined call
// runs its chunks in several launches, in order, the state between them
// exact in f32.
template <int R, bool GATED, int W>
__global__ __launch_bounds__(64 * W) void prefill_chunk_kernel(
    float* __restrict__ state, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int num_slots, int Hk, int T, int plo, int phi,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ vc, const float* __restrict__ lgv,
    const uint16_t* __restrict__ betav, const uint16_t* __restrict__ rec, uint16_t* __restrict__ y,
    const uint16_t* __restrict__ zrow, int64_t xs, const uint16_t* __restrict__ norm_w,
    float norm_eps, uint16_t* __restrict__ out, uint32_t* __restrict__ status) {
  static_assert(W == 2 || W == 4 || W == 8, "8 waves (fused) or a split of 2 or 4");
  static_assert(W == 8 || !GATED, "the split path has no epilogue");
  constexpr bool FUSED = W == 8;
  constexpr int NT = 64 * W;
  constexpr int UK = kC * kDk / 8 / NT;         // 16-byte k (and q) units per thread
  constexpr int UV = 2;                         // 16-byte v units per thread (2W per row)
  constexpr int UR = (kRecUnits + NT - 1) / NT; // 16-byte record units per thread
  constexpr int M = R * (8 / W);                // groups per (sequence, key head)
  __shared__ std::conditional_t<FUSED, ChunkSmem, SplitSmem<W>> sm;
  const int Hv = Hk * R;
  int hv, s, split;
  {
    const int L = blockIdx.x;
    int g, m;
    if ((int)gridDim.x % (8 * M) == 0) {
      m = (L >> 3) % M;
      g = (L & 7) + 8 * ((L >> 3) / M);
    } else {
      m = L % M;
      g = L / M;
    }
    s = g / Hk;
    hv = (g % Hk) * R + m % R;
    split = m / R;
  }
  const int hk = hv / R;
  const int tid = threadIdx.x, lane0 = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave index, scalar
  const int dvb = 16 * W * split;                          // the group's first state row
  const int dv0 = dvb + 16 * w;                            // this wave's first state row
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0 && blockIdx.x == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  if (en <= st || en <= plo || phi <= st) return;
  // the window's chunks: cb = the first one ending past plo, ce = the end of
  // the last one ending at or before phi
  const int cb = plo > st ? st + kC * ((plo - st) / kC) : st;
  const int ce = en > phi ? st + kC * ((phi - st) / kC) : en;
  if (ce <= cb) return;
  const int q0 = lane0 >> 4, c0l = lane0 & 15;
  // this lane's state column (accumulator column c = state row dv0 + c)
  float* gstate = state + (size_t)slot * Hv * kTileElems + state_row_offset(hv, dv0 + c0l, Hk, R) + 4 * q0;
  f32x4 acc[8];  // S^T tiles: dk rows 16a + 4q + r, state row dv0 + c
#pragma unroll
  for (int a = 0; a < 8; ++a) acc[a] = *reinterpret_cast<const f32x4*>(gstate + 16 * a);
  // write-out layout: thread (tokens oi and oi + 32, 8 output rows from od);
  // 2W lanes cover one token's 32W-byte part of the row
  const int oi = tid / (2 * W), od = dvb + 8 * (tid % (2 * W));
  u32x4 nw = {0u, 0u, 0u, 0u};  // GATED: the norm weights of rows od..od+7
  if constexpr (GATED) nw = *reinterpret_cast<const u32x4*>(norm_w + od);
  // Blocks of P above the diagonal are never written: zero them once.
  if constexpr (FUSED)
    for (int e = tid; e < kC * kLdP / 4; e += NT) reinterpret_cast<uint2*>(&sm.P[0][0])[e] = make_uint2(0u, 0u);

  // chunk inputs, prefetched one chunk ahead: 16-byte units of the k, q and
  // v rows (thread e: row e/16, elements 8(e%16)..+7) and, for lane l, token
  // l's beta (raw bf16) and log decay; 8 loads per wave and chunk. A CU
  // passes these 48 KiB per chunk through its texture units at ~64 B per
  // cycle, and a wave that issues into a full queue stalls, so the four
  // groups go out at four points of the chunk (k in (b), q in (c), v in (d),
  // the gates in (e)). Every read goes through a buffer resource whose size
  // ends at the chunk's last token (0 past the window's last chunk: the
  // tokens after it may still be in the making), so rows beyond it read 0
  // without a branch: a load under a branch leaves a merge of
  // its result with the zero of the other path, and the copy that merge needs
  // makes the wave wait for the load right after issuing it instead of one
  // chunk later. Sizes go through readfirstlane: a resource held in VGPRs
  // would need a waterfall loop around each load.
  u32x4 kv[UK], qv[UK], vv[UV], rv[UR];
  uint16_t pb = 0;
  float pl = 0.f;
  auto rows_of = [&](int c) { return __builtin_amdgcn_readfirstlane(max(0, min(kC, ce - c))); };
  // k (KQ = 0) or q (KQ = 1) rows of the chunk at token c
  auto load_kq = [&](int c, auto KQ) {
    const int n = rows_of(c);
    const int bytes = __builtin_amdgcn_readfirstlane(n > 0 ? ((n - 1) * Hk + 1) * kDk * 2 : 0);
    const uint16_t* src = (decltype(KQ)::value ? qn : kn) + ((size_t)c * Hk + hk) * kDk;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, bytes, 0x00020000);
#pragma unroll
    for (int u = 0; u < UK; ++u) {
      const int e = tid + NT * u;
      const int i = decltype(KQ)::value ? qrow(e) : e >> 4, m = decltype(KQ)::value ? qunit(e) : e & 15;
      const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, i * Hk * kDk * 2 + 16 * m, 0, 0);
      if constexpr (decltype(KQ)::value) qv[u] = x; else kv[u] = x;
    }
  };
  // v: the group's 16W columns of the chunk's rows (unit e: row e/(2W),
  // columns dvb + 8(e%(2W)) ..)
  auto load_v = [&](int c) {
    const int n = rows_of(c);
    const int bytes = __builtin_amdgcn_readfirstlane(n > 0 ? ((n - 1) * Hv + 1) * kDv * 2 - 2 * dvb : 0);
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(vc + ((size_t)c * Hv + hv) * kDv + dvb), (short)0, bytes, 0x00020000);
#pragma unroll
    for (int u = 0; u < UV; ++u) {
      const int e = tid + NT * u, i = e / (2 * W), m = e % (2 * W);
      vv[u] = __builtin_amdgcn_raw_buffer_load_b128(r, i * Hv * kDv * 2 + 16 * m, 0, 0);
    }
  };
  // split path: the record of the chunk at token c (none past the sequence end)
  auto load_rec = [&](int c) {
    const int n = rows_of(c);
    const int x = st / kC + s + (c - st) / kC;
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(rec + ((size_t)x * Hv + hv) * (kRecBytes / 2)), (short)0, n > 0 ? kRecUnits * 16 : 0,
        0x00020000);
#pragma unroll
    for (int j = 0; j < UR; ++j) rv[j] = __builtin_amdgcn_raw_buffer_load_b128(r, 16 * (tid + NT * j), 0, 0);
  };
  // every wave reads the 64 gate values (wave 0 uses them)
  auto load_gates = [&](int c) {
    const int n = rows_of(c);
    const int g = __builtin_amdgcn_readfirstlane(n > 0 ? (n - 1) * Hv + 1 : 0);
    const __amdgpu_buffer_rsrc_t br = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(betav + (size_t)c * Hv + hv), (short)0, 2 * g, 0x00020000);
    const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)(lgv + (size_t)c * Hv + hv), (short)0, 4 * g, 0x00020000);
    pb = __builtin_amdgcn_raw_buffer_load_b16(br, lane0 * Hv * 2, 0, 0);
    pl = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(lr, lane0 * Hv * 4, 0, 0));
  };
  // split path: the LDS byte offsets of this thread's record units, the same
  // for every chunk
  uint32_t roff[FUSED ? 1 : UR];
  if constexpr (!FUSED) {
#pragma unroll
    for (int j = 0; j < UR; ++j) {
      const int u = min(tid + NT * j, kRecUnits - 1);
      roff[j] = static_cast<uint32_t>(static_cast<char*>(rec_slot(sm, u)) - reinterpret_cast<char*>(&sm));
    }
  }
  using KLoad = std::integral_constant<int, 0>;
  using QLoad = std::integral_constant<int, 1>;
  // Without the gated epilogue a chunk's outputs (step (e)) are formed during
  // the next chunk's products, where the SIMDs have issue slots to spare
  // (most on the split path, one wave per SIMD), from the chunk's Zt, V'h, P
  // fragments and exp(G) kept in registers, and written out after that
  // chunk's closing barrier; the last chunk's after the loop. The same
  // products in the same order: the same bits. (The gated epilogue also
  // needs every wave's sums of y^2 and z: it stays in its own chunk.)
  constexpr bool DEFER = !GATED;
  f32x4 ztp[DEFER ? 4 : 1];   // Zt of the previous chunk
  s16x4 vpp[DEFER ? 4 : 1];   // its V'h
  bf16x8 ppp[DEFER ? 6 : 1];  // its P fragments: rows 16I + c, pairs p <= I / 2
  float egp[DEFER ? 4 : 1];   // exp(G) of its tokens 16I + c
  int cp = -1, np = 0;        // its first token and rows (cp < 0: none yet)
  auto out_prev = [&]() {
    int k = 0;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 o = ztp[I] * egp[I];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (2 * p > I) continue;
        o = mfma32(cat(vpp[2 * p], vpp[2 * p + 1]), ppp[k++], o);
      }
      *reinterpret_cast<uint2*>(&sm.Y[16 * I + c0l][16 * w + 4 * q0]) =
          make_uint2(f2bf2(o[0], o[1]), f2bf2(o[2], o[3]));
    }
  };
  // write-out of the chunk at token cx (rows nx) from the LDS rows of y:
  // thread (tokens oi and oi + 32, rows od..od+7), 16 bytes of y per token
  auto write_out = [&](int cx, int nx) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int i = oi + 32 * h;
      if (i >= nx) continue;
      const uint2 ya = *reinterpret_cast<const uint2*>(&sm.Y[i][od - dvb]);
      const uint2 yb = *reinterpret_cast<const uint2*>(&sm.Y[i][od - dvb + 4]);
      *reinterpret_cast<uint4*>(y + ((size_t)(cx + i) * Hv + hv) * kDv + od) =
          make_uint4(ya.x, ya.y, yb.x, yb.y);
    }
  };
  load_kq(cb, KLoad{});
  load_kq(cb, QLoad{});
  load_v(cb);
  if constexpr (FUSED) load_gates(cb); else load_rec(cb);
  for (int c0 = cb; c0 < ce; c0 += kC) {
    const int n = min(kC, en - c0);
    // Lane-derived values are recomputed in every chunk (a few VALU ops)
    // instead of being held in registers across the loop.
    int lane = lane0;
    asm volatile("" : "+v"(lane));
    const int q = lane >> 4, c = lane & 15;
    const int kf = kseg(c, q), kt = kseg(4 * q + (c >> 2), c & 3);  // K operand lane constants
    const int qs = 8 * (q ^ gsw(c));  // column of this lane's 16-byte group q in rows of NL and P
    // (a) stage k (natural order, swizzled segments), q (pair order) and v;
    // wave 0 forms the decay prefix sums in log2 units
#pragma unroll
    for (int u = 0; u < UK; ++u) {
      // k: natural segments 2m, 2m + 1 stay adjacent and in order under the
      // (even) swizzle, one 16-byte write
      const int e = tid + NT * u, i = e >> 4, m = e & 15;
      *static_cast<u32x4*>(__builtin_assume_aligned(&sm.K[kseg(i, 2 * m)], 16)) = kv[u];
      // q (unit qunit(e) of row qrow(e)): dk 8m..8m+3 and 8m+4..8m+7 go to
      // pair-order places p and p + 8, p = 32(m/4) + 16(m%2) + 4((m/2)%2).
      // An 8-byte write pass (16 lanes) covers units 0-7 or 8-15 of an even
      // and the next odd row; the odd row writes its second half first, which
      // puts the 16 writes in 32 distinct banks.
      const int qi = qrow(e), qm = qunit(e);
      const int p = 32 * (qm >> 2) + 16 * (qm & 1) + 4 * ((qm >> 1) & 1), odd = qi & 1;
      const u32x2 qlo = {qv[u][0], qv[u][1]}, qhi = {qv[u][2], qv[u][3]};
      *static_cast<u32x2*>(__builtin_assume_aligned(&sm.Q[qi][p + 8 * odd], 8)) = odd ? qhi : qlo;
      *static_cast<u32x2*>(__builtin_assume_aligned(&sm.Q[qi][p + 8 - 8 * odd], 8)) = odd ? qlo : qhi;
    }
#pragma unroll
    for (int u = 0; u < UV; ++u) {
      const int e = tid + NT * u, i = e / (2 * W), m = e % (2 * W);
      *static_cast<u32x4*>(__builtin_assume_aligned(&sm.V[i][8 * m], 16)) = vv[u];
    }
    if constexpr (FUSED) {
      if (w == 0) form_gates(sm, pb, pl, lane0);
    } else {
#pragma unroll
      for (int j = 0; j < UR; ++j)
        if (tid + NT * j < kRecUnits)
          *static_cast<u32x4*>(__builtin_assume_aligned(reinterpret_cast<char*>(&sm) + roff[j], 16)) = rv[j];
    }
    __syncthreads();
    load_kq(c0 + kC, KLoad{});  // past the window: no memory access, reads 0
    if constexpr (DEFER)
      if (cp >= 0) out_prev();  // the previous chunk's outputs into the LDS rows of y

    if constexpr (FUSED) {
      // (b) the chunk's matrices: waves 0-3 the diagonal blocks of L and their
      // inverses, waves 4-7 the other 16 blocks of L and P
#pragma unroll
      for (int I = 0; I < 4; ++I)
        if (w == I) invert_diag(sm, I, kf, q, c, lane0);  // block index a compile-time constant
      other_blocks(sm, w, kf, q, c);
    }
    load_kq(c0 + kC, QLoad{});
    // (c) Y_I = K_I S^T (S hi and lo) and Zt_I = S Q_I^T (S hi) for this wave's
    // 16 state rows; the pair (acc[2b], acc[2b+1]) is the operand of dk block b
    f32x4 yk[4], zt[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      yk[I] = f32x4{0.f, 0.f, 0.f, 0.f};
      zt[I] = yk[I];
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      // fused: bound live ranges, one dk block at a time (two waves per SIMD
      // share its registers); the split path has the registers to keep every
      // block's operand reads in flight together
      if constexpr (FUSED) asm volatile("" ::: "memory");
      s16x4 h0, l0, h1, l1;
      split4(acc[2 * b], h0, l0);
      split4(acc[2 * b + 1], h1, l1);
      const bf16x8 sh = cat(h0, h1), sl = cat(l0, l1);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const bf16x8 ka = kfrag(sm.K, kf, I, b);
        yk[I] = mfma32(ka, sh, yk[I]);
        yk[I] = mfma32(ka, sl, yk[I]);
        zt[I] = mfma32(sh, lds8(&sm.Q[16 * I + c][32 * b + 8 * q]), zt[I]);
      }
    }
    if constexpr (FUSED) __syncthreads();  // the blocks formed in (b)

    load_v(c0 + kC);
    // (d) R_I = beta (V - exp(G) Y_I), then V'_I = D_I (R_I - sum_{j<I} L_Ij V'_j),
    // right-looking: as soon as V'_I is known it is added into the right-hand
    // sides of the blocks below it, so the chain between two blocks is two
    // MFMAs, not all of the later block's terms. Each x_J still adds its terms
    // in the order R_J, j = 0, 1, ..
    f32x4 x[4];         // right-hand sides, tokens 16I + 4q + r, state row dv0 + c
    f32x4 vf[4];        // V' (f32)
    s16x4 vph[4];       // V'h
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const f32x4 bt = *reinterpret_cast<const f32x4*>(&sm.beta[16 * I + 4 * q]);
      const f32x4 eg = *reinterpret_cast<const f32x4*>(&sm.eG[16 * I + 4 * q]);
      // v of tokens 16I + 4q + r, state row dv0 + c (a transposing read: lane
      // 4u + s of each 16-lane group reads row 4q + u, columns 4s..4s+3)
      const s16x4 vt = vtr(sm, 16 * I + 4 * q + (c >> 2), 16 * w + 4 * (c & 3));
#pragma unroll
      for (int r = 0; r < 4; ++r) x[I][r] = bt[r] * fmaf(-eg[r], yk[I][r], bf2f((uint16_t)vt[r]));
    }
    // (f) on the split path, first half: S^T <- exp(G_C) S^T + K^T (exp(G_C -
    // G) V'), V' hi and lo, for tokens 32p .. 32p + 31 (acc[a] takes p = 0 hi,
    // lo, then p = 1 hi, lo, as in the fused path's (f)). The p = 0 half goes
    // out as soon as blocks 0 and 1 of V' are known, so that its MFMAs fill
    // the dependent chain of blocks 2 and 3: a group of W <= 4 waves has one
    // wave per SIMD, with nothing else to issue there. (The fused path's two
    // waves per SIMD already fill it: the same order measured no faster.)
    auto update_half = [&](int p) {
      s16x4 h0, l0, h1, l1;
      const f32x4 d0 = *reinterpret_cast<const f32x4*>(&sm.dec[32 * p + 4 * q]);
      const f32x4 d1 = *reinterpret_cast<const f32x4*>(&sm.dec[32 * p + 16 + 4 * q]);
      split4(vf[2 * p] * d0, h0, l0);
      split4(vf[2 * p + 1] * d1, h1, l1);
      const bf16x8 vth = cat(h0, h1), vtl = cat(l0, l1);
      if (p == 0) {
        const float eC = sm.eG[kC - 1];
#pragma unroll
        for (int a = 0; a < 8; ++a) acc[a] *= eC;
      }
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        const bf16x8 ka = cat(ktr(sm.K, kt, 2 * p, a), ktr(sm.K, kt, 2 * p + 1, a));
        acc[a] = mfma32(ka, vth, acc[a]);
        acc[a] = mfma32(ka, vtl, acc[a]);
      }
    };
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      s16x4 xh, xl;
      split4(x[I], xh, xl);
      const bf16x8 d = lds8(&sm.D[I * kLdDB + c * kLdD + 8 * q]);  // D hi | lo
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      v = mfma32(d, cat(xh, xh), v);     // (Dh + Dl) xh
      v = mfma32(d, cat(xl, kZero4), v); // Dh xl
      vf[I] = v;
      s16x4 vl;
      split4(v, vph[I], vl);
      const bf16x8 vpd = cat(vph[I], vph[I]), vplz = cat(vl, kZero4);
#pragma unroll
      for (int J = I + 1; J < 4; ++J) {
        const bf16x8 nl = lds8(nl_row(sm, 16 * J + c) + 32 * I + qs);  // -L_JI hi | lo
        x[J] = mfma32(nl, vpd, x[J]);   // (NLh + NLl) V'h
        x[J] = mfma32(nl, vplz, x[J]);  // NLh V'l
      }
      if (!FUSED && I == 1) update_half(0);
    }
    if constexpr (FUSED) load_gates(c0 + kC); else load_rec(c0 + kC);
    // GATED: z of this thread's two write-out tokens of this chunk, read here
    // so that it arrives during (e) and (f); a token past the chunk's end
    // reads the chunk's last row instead (its output is not written), which
    // keeps the loads unconditional
    u32x4 zv[2];
    if constexpr (GATED) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int i = min(oi + 32 * h, n - 1);
        zv[h] = *reinterpret_cast<const u32x4*>(zrow + (size_t)(c0 + i) * xs + (size_t)hv * kDv + od);
      }
    }
    // (e) O^T_I = exp(G) Zt_I + V'^T P^T: rows dv0 + 4q + r, token 16I + c
    // y (bf16) into the LDS rows; with GATED each wave's sum of y^2 per token.
    // Without GATED the operands are kept for the next chunk instead.
    if constexpr (DEFER) {
      int k = 0;
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        ztp[I] = zt[I];
        vpp[I] = vph[I];
        egp[I] = sm.eG[16 * I + c];
#pragma unroll
        for (int p = 0; p < 2; ++p)
          if (2 * p <= I) ppp[k++] = lds8(&sm.P[16 * I + c][32 * p + qs]);
      }
    }
#pragma unroll
    for (int I = 0; I < (DEFER ? 0 : 4); ++I) {
      f32x4 o = zt[I] * sm.eG[16 * I + c];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        if (2 * p > I) continue;
        o = mfma32(cat(vph[2 * p], vph[2 * p + 1]), lds8(&sm.P[16 * I + c][32 * p + qs]), o);
      }
      const uint2 yb = make_uint2(f2bf2(o[0], o[1]), f2bf2(o[2], o[3]));
      *reinterpret_cast<uint2*>(&sm.Y[16 * I + c][16 * w + 4 * q]) = yb;
      if constexpr (GATED) {
        float ss = sumsq4(bf_lo(yb.x), bf_hi(yb.x), bf_lo(yb.y), bf_hi(yb.y));
        ss += __shfl_xor(ss, 16, 64);
        ss += __shfl_xor(ss, 32, 64);
        if (q == 0) sm.ysq[16 * I + c][w] = ss;
      }
    }
    // (f) S^T <- exp(G_C) S^T + K^T (exp(G_C - G) V'), V' hi and lo
    if constexpr (FUSED) {
      bf16x8 vth[2], vtl[2];
#pragma unroll
      for (int p = 0; p < 2; ++p) {
        s16x4 h0, l0, h1, l1;
        const f32x4 d0 = *reinterpret_cast<const f32x4*>(&sm.dec[32 * p + 4 * q]);
        const f32x4 d1 = *reinterpret_cast<const f32x4*>(&sm.dec[32 * p + 16 + 4 * q]);
        split4(vf[2 * p] * d0, h0, l0);
        split4(vf[2 * p + 1] * d1, h1, l1);
        vth[p] = cat(h0, h1);
        vtl[p] = cat(l0, l1);
      }
      const float eC = sm.eG[kC - 1];
#pragma unroll
      for (int a = 0; a < 8; ++a) {
        acc[a] *= eC;
#pragma unroll
        for (int p = 0; p < 2; ++p) {
          const bf16x8 ka = cat(ktr(sm.K, kt, 2 * p, a), ktr(sm.K, kt, 2 * p + 1, a));
          acc[a] = mfma32(ka, vth[p], acc[a]);
          acc[a] = mfma32(ka, vtl[p], acc[a]);
        }
      }
    } else {
      update_half(1);  // second half: tokens 32 .. 63
    }
    __syncthreads();
    if constexpr (DEFER) {  // (g) of the previous chunk, whose rows out_prev formed
      if (cp >= 0 && y != nullptr) write_out(cp, np);
      cp = c0;
      np = n;
    }
    // (g) write-out: thread (tokens oi and oi + 32, rows od..od+7) stores 16
    // bytes of y per token; GATED: out = silu(z) * bf16(w * bf16(y * rn)), rn
    // from the 8 waves' sums of y^2
#pragma unroll
    for (int h = 0; h < (DEFER ? 0 : 2); ++h) {
      const int i = oi + 32 * h;
      if (i >= n) continue;
      const uint2 ya = *reinterpret_cast<const uint2*>(&sm.Y[i][od - dvb]);
      const uint2 yb = *reinterpret_cast<const uint2*>(&sm.Y[i][od - dvb + 4]);
      const uint4 yv = make_uint4(ya.x, ya.y, yb.x, yb.y);
      const size_t row = ((size_t)(c0 + i) * Hv + hv) * kDv + od;
      if (y != nullptr) *reinterpret_cast<uint4*>(y + row) = yv;
      if constexpr (GATED) {
        const f32x4 p0 = *reinterpret_cast<const f32x4*>(&sm.ysq[i][0]);
        const f32x4 p1 = *reinterpret_cast<const f32x4*>(&sm.ysq[i][4]);
        const float tot = ((p0[0] + p0[1]) + (p0[2] + p0[3])) + ((p1[0] + p1[1]) + (p1[2] + p1[3]));
        const u32x4 o = norm_gate8(u32x4{yv.x, yv.y, yv.z, yv.w}, zv[h], nw, rms_scale(tot, norm_eps));
        *reinterpret_cast<u32x4*>(out + row) = o;
      }
    }
  }
  if constexpr (DEFER) {  // the last chunk's outputs
    __syncthreads();  // every wave's reads of the LDS rows of y are done
    out_prev();
    __syncthreads();
    if (y != nullptr) write_out(cp, np);
  }
#pragma unroll
  for (int a = 0; a < 8; ++a)
    *reinterpret_cast<f32x4*>(gstate + 16 * a) = acc[a];
}

// Shared memory of prefill_form_kernel: the block-forming part of ChunkSmem.
struct __attribute__((aligned(16))) FormSmem {
  static constexpr int kNLRow0 = 16;  // block row 0 of -L holds no record block
  uint16_t K[4 * kKBlk];
  uint16_t Q[kC][kLdQ];
  uint16_t P[kC][kLdP];
  uint16_t NL[kC - 16][kLdN];
  uint16_t D[4 * kLdDB];
  float Ld[4 * kLdLB];
  float beta[kC], G[kC], eG[kC], dec[kC];
};

// Split path, step 1 of 2: for every (chunk, value head) of the call at once,
// the chunk's blocks of L and P, the inverses D_I and the gates, formed by the
// same code as in the chunk kernel's step (b), written as the chunk's record
// (see rec_slot). Item = (record slot x0 + item / Hv, value head); slots
// that hold no chunk (see rec_slots), and chunks whose last token + 1 lies
// outside (plo, phi], exit. 8 waves: waves 0-3 invert the diagonal blocks,
// waves 4-7 form the other 16. The R heads of one (slot, key head) are
// numbered 8 apart, so they run on one XCD and share its k and q rows.
template <int R>
__global__ __launch_bounds__(512) void prefill_form_kernel(
    const int32_t* __restrict__ cu, int nseq, int Hk, int T, int x0, int plo, int phi,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const float* __restrict__ lgv, const uint16_t* __restrict__ betav, uint16_t* __restrict__ rec) {
  constexpr int NT = 512;
  __shared__ FormSmem sm;
  const int Hv = Hk * R;
  int g, r;
  {
    const int L = blockIdx.x;
    if ((int)gridDim.x % (8 * R) == 0) {
      const int m = L >> 3;
      g = (L & 7) + 8 * (m / R);
      r = m % R;
    } else {
      g = L / R;
      r = L % R;
    }
  }
  const int x = x0 + g / Hk, hk = g % Hk, hv = hk * R + r;
  // the sequence of slot x: the largest s with floor(st_s / 64) + s <= x
  int lo = 0, hi = nseq - 1;
  while (lo < hi) {
    const int mid = (lo + hi + 1) >> 1;
    if (min(max(cu[mid], 0), T) / kC + mid <= x) lo = mid; else hi = mid - 1;
  }
  const int s = lo;
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  // (a slot below the sequence's first one only with a malformed cu_seqlens)
  if (x < st / kC + s) return;
  const int c0 = st + kC * (x - st / kC - s);
  if (c0 >= en) return;
  const int n = min(kC, en - c0);
  if (c0 + n <= plo || c0 + n > phi) return;  // another segment's chunk
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int q = lane >> 4, c = lane & 15, kf = kseg(c, q);
  // P's halves above the diagonal belong to the record: zero P first
  for (int e = tid; e < kC * kLdP / 4; e += NT) reinterpret_cast<uint2*>(&sm.P[0][0])[e] = make_uint2(0u, 0u);
  // k (natural order, swizzled segments) and q (pair order) of the chunk's
  // rows, 0 beyond its last token; two 16-byte units per thread and matrix
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int e = tid + NT * u, i = e >> 4, m = e & 15;
    u32x4 kv = {0u, 0u, 0u, 0u}, qv = kv;
    if (i < n) {
      const size_t row = ((size_t)(c0 + i) * Hk + hk) * kDk;
      kv = *reinterpret_cast<const u32x4*>(kn + row + 8 * m);
      qv = *reinterpret_cast<const u32x4*>(qn + row + 8 * m);
    }
    *static_cast<u32x4*>(__builtin_assume_aligned(&sm.K[kseg(i, 2 * m)], 16)) = kv;
    const int p = 32 * (m >> 2) + 16 * (m & 1) + 4 * ((m >> 1) & 1);
    *static_cast<u32x2*>(__builtin_assume_aligned(&sm.Q[i][p], 8)) = u32x2{qv[0], qv[1]};
    *static_cast<u32x2*>(__builtin_assume_aligned(&sm.Q[i][p + 8], 8)) = u32x2{qv[2], qv[3]};
  }
  if (w == 0) {
    uint16_t b = 0;
    float lg = 0.f;
    if (lane < n) {
      b = betav[(size_t)(c0 + lane) * Hv + hv];
      lg = lgv[(size_t)(c0 + lane) * Hv + hv];
    }
    form_gates(sm, b, lg, lane);
  }
  __syncthreads();
#pragma unroll
  for (int I = 0; I < 4; ++I)
    if (w == I) invert_diag(sm, I, kf, q, c, lane);
  other_blocks(sm, w, kf, q, c);
  __syncthreads();
  uint16_t* dst = rec + ((size_t)x * Hv + hv) * (kRecBytes / 2);
  for (int u = tid; u < kRecUnits; u += NT)
    *reinterpret_cast<u32x4*>(dst + 8 * u) = *static_cast<const u32x4*>(__builtin_assume_aligned(rec_slot(sm, u), 16));
}

// Split path, RMSNormGated epilogue (qwen3_5.rs:660-665) over y written by the
// chunk kernel: out[t, hv, :] = silu(z) * bf16(w * bf16(y * rn)). 16 lanes per
// (token, value head), lane j rows 8j..8j+7; the sum of y^2 runs in the order
// of the chunk kernel's own epilogue (per 4 rows, then per 16, then over the
// 8 groups of 16 pairwise), so that both paths give the same bits.
__global__ __launch_bounds__(256) void prefill_norm_gate_kernel(
    const uint16_t* __restrict__ y, const uint16_t* __restrict__ zrow, int64_t xs,
    const uint16_t* __restrict__ norm_w, float norm_eps, uint16_t* __restrict__ out, int T, int Hv) {
  const int item = blockIdx.x * 16 + (threadIdx.x >> 4), j = threadIdx.x & 15;
  if (item >= T * Hv) return;  // a whole 16-lane group
  const int t = item / Hv, hv = item % Hv;
  const size_t row = ((size_t)t * Hv + hv) * kDv + 8 * j;
  const u32x4 yv = *reinterpret_cast<const u32x4*>(y + row);
  const u32x4 zv = *reinterpret_cast<const u32x4*>(zrow + (size_t)t * xs + (size_t)hv * kDv + 8 * j);
  const u32x4 nw = *reinterpret_cast<const u32x4*>(norm_w + 8 * j);
  // lane 2k: rows 16k..16k+7 (the chunk kernel's lanes q = 0, 1 of wave k),
  // lane 2k + 1: rows 16k+8..16k+15 (q = 2, 3)
  float p = sumsq4(bf_lo(yv[0]), bf_hi(yv[0]), bf_lo(yv[1]), bf_hi(yv[1])) +
            sumsq4(bf_lo(yv[2]), bf_hi(yv[2]), bf_lo(yv[3]), bf_hi(yv[3]));
  p = sum16(p);  // xor 1, 2, 4, 8 partner order on DPP
  *reinterpret_cast<u32x4*>(out + row) = norm_gate8(yv, zv, nw, rms_scale(p, norm_eps));
}

// Waves per work-group of the chunk kernel for a call: 8 runs the fused
// chunk kernel alone (one group per (sequence, value head)); 2 or 4 run the
// split path (prefill_form_kernel, then 8/W groups per (sequence, value
// head)) where the fused kernel would leave most CUs idle: few sequences of
// many chunks. The environment variable GDN_PREFILL_WAVES = 2, 4 or 8 forces
// a path (tests compare the paths with it).
// The path GDN_PREFILL_WAVES forces (2, 4 or 8), or 0.
static int forced_chunk_waves() {
  if (const char* v = getenv("GDN_PREFILL_WAVES")) {
    const int f = atoi(v);
    if (f == 2 || f == 4 || f == 8) return f;
  }
  return 0;
}

int prefill_chunk_waves(int R, int Hk, int nseq, int total_tokens) {
  if (const int f = forced_chunk_waves()) return total_tokens > 0 ? f : 8;
  if (nseq <= 0 || total_tokens <= 0 || total_tokens > kSplitMaxTokens) return 8;
  if (total_tokens / nseq < kSplitMinTokens) return 8;
  // measured on 16,384-token prompts (32 value heads): one or two prompts
  // 1.10 / 1.30 ms split against 1.36 / 1.50 ms fused per call; four prompts
  // 1.80 ms with 4-wave groups against 1.76 ms fused
  const int groups = nseq * Hk * R;
  return groups <= 64 ? 2 : groups <= 96 ? 4 : 8;
}

// When the split path's chunk kernel leaves at least half of the CUs idle (its
// groups, one per CU, number at most half the CUs), a call of at least two
// segments of kPipeSegmentTokens runs its qkv and form kernels one segment
// ahead on a second stream, beside the chunk kernel of the previous segment.
// At 32 value heads that admits one prompt. Pipelining several long prompts
// loses: segments cut the packed tokens, so a later prompt falls wholly into
// the last segments and its chain starts only after the first prompt's (two
// 16,384-token prompts forced into segments: 1.72-1.75 ms per layer at 256
// 2-wave groups, 1.68-1.72 at 128 4-wave groups, against 1.19 in one pass).
// GDN_PREFILL_SEGMENTS = n forces n segments (1: one pass) on the split path.
constexpr int kPipeSegmentTokens = 4096;

int prefill_pipeline_segments(int waves, int total_tokens, int groups, int cus) {
  if (waves != 2 && waves != 4) return 1;
  if ((waves != 2 || 2 * (int64_t)groups > cus) && !getenv("GDN_PREFILL_SEGMENTS")) return 1;
  const int tiles = (total_tokens + kTT - 1) / kTT;
  int n = total_tokens / kPipeSegmentTokens;
  if (const char* v = getenv("GDN_PREFILL_SEGMENTS")) n = atoi(v);
  return std::max(1, std::min({n, kPrefillPipeSegmentsMax, tiles}));
}

size_t prefill_workspace_bytes(int R, int Hk, int total_tokens, int nseq, int waves, bool y_scratch) {
  return carve(nullptr, R, Hk, total_tokens, nseq, waves, y_scratch, nullptr);
}

size_t prefill_workspace_reserve_bytes(int R, int Hk, int max_tokens) {
  // the largest call the split path takes: every sequence count it picks,
  // the gated epilogue's y scratch included
  size_t most = prefill_workspace_bytes(R, Hk, max_tokens, 1, 8, false);
  // a forced split takes any call: up to one sequence per token
  const int f = forced_chunk_waves();
  if (f == 2 || f == 4)
    most = std::max(most, prefill_workspace_bytes(R, Hk, max_tokens, std::max(max_tokens, 1), f,
                                                  true));
  if (max_tokens > kSplitMaxTokens) max_tokens = kSplitMaxTokens;
  for (int nseq = 1; nseq * Hk * R <= 96 && nseq <= max_tokens; ++nseq)
    most = std::max(most, prefill_workspace_bytes(R, Hk, max_tokens, nseq, 2, true));
  return most;
}

// ---------------------------------------------------- no-allocation scratch --
// Workspace of gdn_prefill_varlen_noalloc: one fixed array per device, in
// place of the pool's grown workspace. Every call on a device shares it and
// finds the previous call's contents (the prefill writes every workspace byte
// it reads, so nothing needs clearing); calls that overlap on one device race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
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

// Split path with out: the RMSNormGated epilogue over y.
static hipError_t launch_split_norm_gate(const PrefillArgs& a, const uint16_t* yb) {
  const int Hv = a.Hk * a.R;
  const int D = 2 * a.Hk * kDk + Hv * kDv;
  const long items = (long)a.total_tokens * Hv;
  hipLaunchKernelGGL(prefill_norm_gate_kernel, dim3((unsigned)((items + 15) / 16)), dim3(256), 0,
                     a.stream, yb, a.mixed + D, a.xstride, a.norm_w, a.norm_eps, a.out,
                     a.total_tokens, Hv);
  return hipGetLastError();
}

template <int R, int W>
static hipError_t launch_split(const PrefillArgs& a, const Workspace& ws) {
  const int Hv = a.Hk * R;
  hipLaunchKernelGGL(prefill_form_kernel<R>, dim3(rec_slots(a.total_tokens, a.nseq) * Hv), dim3(512),
                     0, a.stream, a.cu_seqlens, a.nseq, a.Hk, a.total_tokens, 0, 0, a.total_tokens,
                     ws.qn, ws.kn, ws.lg, ws.beta, ws.rec);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  uint16_t* yb = a.y ? a.y : ws.y;
  hipLaunchKernelGGL((prefill_chunk_kernel<R, false, W>), dim3(Hv * a.nseq * (8 / W)), dim3(64 * W), 0,
                     a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, a.total_tokens,
                     0, a.total_tokens, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, ws.rec, yb, nullptr,
                     a.xstride, nullptr, 0.0f, nullptr, a.status);
  e = hipGetLastError();
  if (e != hipSuccess || !a.out) return e;
  return launch_split_norm_gate(a, yb);
}

// The split path in `segs` segments of whole 64-token tiles, each twice the
// one before: segment 0 is short, so little of its qkv and form work is
// exposed, and each later segment's qkv and form kernels (on the second
// stream) take less time than the chunk kernel of the segment before, beside
// which they run (one 16,384-token prompt, 4 segments: 0.930 ms per layer
// with growth 2, 0.937-0.944 with 1.5-1.75 or 2.25, 0.969-0.986 with 3-4,
// 0.973 with equal segments, 1.022 in one pass).
// Segment 0's kernels go to the caller's stream (no cross-stream wait ahead
// of them), and the second stream starts once segment 0's qkv kernel is done
// (a chunk of segment 1 may begin in segment 0's tokens, and the conv-state
// update must follow every read of the old rows); segment j >= 1's chunk
// kernel waits for its qkv and form kernels on the caller's stream. The
// conv-state update follows the last qkv kernel on the second stream, and the
// caller's stream waits for it. Every kernel does the same arithmetic as in
// one pass: the same bits.
static int pipeline_tile(int tiles, int segs, int j) {
  // tiles * (2^j - 1) / (2^segs - 1), every segment at least one tile
  const int t = (int)((int64_t)tiles * ((1 << j) - 1) / ((1 << segs) - 1));
  return std::min(std::max(t, j), tiles - (segs - j));
}

template <int R, int W>
static hipError_t launch_split_pipelined(const PrefillArgs& a, const Workspace& ws, int segs) {
  const int Hv = a.Hk * R;
  const int D = 2 * a.Hk * kDk + Hv * kDv;
  const int T = a.total_tokens, tiles = (T + kTT - 1) / kTT;
  const int slots = rec_slots(T, a.nseq);
  uint16_t* yb = a.y ? a.y : ws.y;
  hipEvent_t* ev = a.events;
  hipError_t e = hipSuccess;
  for (int j = 0; j < segs && e == hipSuccess; ++j) {
    const int t0 = pipeline_tile(tiles, segs, j), t1 = pipeline_tile(tiles, segs, j + 1);
    const int plo = t0 * kTT, phi = j + 1 == segs ? T : t1 * kTT;
    hipStream_t sq = j == 0 ? a.stream : a.aux;
    hipLaunchKernelGGL(prefill_qkv_kernel<R>, dim3(2 * a.Hk + Hv, t1 - t0), dim3(256), 0, sq,
                       a.conv, a.slot_ids, a.cu_seqlens, a.nseq, a.num_slots, a.Hk, T, t0, a.mixed,
                       a.xstride, a.conv_w, a.ab, a.ab_stride, a.A_log, a.dt_bias, ws.qn, ws.kn,
                       ws.vc, ws.beta, ws.lg);
    if (j == 0) {  // the second stream starts after segment 0's qkv kernel
      e = hipGetLastError();
      if (e == hipSuccess) e = hipEventRecord(ev[0], a.stream);
      if (e == hipSuccess) e = hipStreamWaitEvent(a.aux, ev[0], 0);
      if (e != hipSuccess) break;
    }
    // record slots of the chunks ending in (plo, phi]: the chunk starts lie
    // in (plo - 64, phi), slot = floor(start / 64) + its sequence
    const int x0 = plo >= kTT ? (plo - kTT + 1) / kTT : 0;
    const int x1 = std::min(slots, (phi - 1) / kTT + a.nseq);
    if (x1 > x0)
      hipLaunchKernelGGL(prefill_form_kernel<R>, dim3((x1 - x0) * Hv), dim3(512), 0, sq,
                         a.cu_seqlens, a.nseq, a.Hk, T, x0, plo, phi, ws.qn, ws.kn, ws.lg, ws.beta,
                         ws.rec);
    e = hipGetLastError();
    if (j > 0) {
      if (e == hipSuccess) e = hipEventRecord(ev[1 + j], a.aux);
      if (e == hipSuccess) e = hipStreamWaitEvent(a.stream, ev[1 + j], 0);
    }
    if (e != hipSuccess) break;
    hipLaunchKernelGGL((prefill_chunk_kernel<R, false, W>), dim3(Hv * a.nseq * (8 / W)), dim3(64 * W),
                       0, a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, T, plo,
                       phi, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, ws.rec, yb, nullptr, a.xstride,
                       nullptr, 0.0f, nullptr, a.status);
    e = hipGetLastError();
  }
  if (e == hipSuccess) {
    hipLaunchKernelGGL(prefill_conv_state_kernel, dim3(a.nseq, (D + 255) / 256), dim3(256), 0,
                       a.aux, a.conv, a.slot_ids, a.cu_seqlens, a.nseq, a.num_slots, D, T, a.mixed,
                       a.xstride, a.status);
    e = hipGetLastError();
  }
  // the caller's stream waits for the second stream's work, also after an
  // error, so that no later call on the pool overlaps what was queued there
  hipError_t j = hipEventRecord(ev[1 + segs], a.aux);
  if (j == hipSuccess) j = hipStreamWaitEvent(a.stream, ev[1 + segs], 0);
  if (e == hipSuccess) e = j;
  if (e != hipSuccess || !a.out) return e;
  return launch_split_norm_gate(a, yb);
}

template <int R>
static hipError_t launch_prefill_r(const PrefillArgs& a) {
  const int Hv = a.Hk * R;
  const int D = 2 * a.Hk * kDk + Hv * kDv;
  Workspace ws;
  carve(a.workspace, R, a.Hk, a.total_tokens, a.nseq, a.waves, a.out && !a.y, &ws);
  const int segs = a.aux && a.events ? a.segments : 1;
  if (segs > 1) {
    if (a.waves == 2) return launch_split_pipelined<R, 2>(a, ws, segs);
    return launch_split_pipelined<R, 4>(a, ws, segs);
  }
  if (a.total_tokens > 0) {
    hipLaunchKernelGGL(prefill_qkv_kernel<R>, dim3(2 * a.Hk + Hv, (a.total_tokens + kTT - 1) / kTT),
                       dim3(256), 0, a.stream, a.conv, a.slot_ids, a.cu_seqlens, a.nseq,
                       a.num_slots, a.Hk, a.total_tokens, 0, a.mixed, a.xstride, a.conv_w, a.ab,
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
  if (a.waves == 2) return launch_split<R, 2>(a, ws);
  if (a.waves == 4) return launch_split<R, 4>(a, ws);
  const int units = Hv * a.nseq;
  if (a.out)
    hipLaunchKernelGGL((prefill_chunk_kernel<R, true, 8>), dim3(units), dim3(512), 0, a.stream,
                       a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, a.total_tokens, 0,
                       a.total_tokens, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, nullptr, a.y,
                       a.mixed + D, a.xstride, a.norm_w, a.norm_eps, a.out, a.status);
  else
    hipLaunchKernelGGL((prefill_chunk_kernel<R, false, 8>), dim3(units), dim3(512), 0, a.stream,
                       a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, a.total_tokens, 0,
                       a.total_tokens, ws.qn, ws.kn, ws.vc, ws.lg, ws.beta, nullptr, a.y, nullptr,
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
