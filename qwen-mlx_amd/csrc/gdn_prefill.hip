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
//   4. chunk_kernel      chunked WY-form recurrence on bf16 MFMA
// Workspace layout (each region 256-byte aligned):
//   xc [T,D] bf16 | qn [T,Hk,Dk] bf16 | kn [T,Hk,Dk] bf16 | beta [T,Hv] bf16 | lg [T,Hv] f32

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
  float* lg;
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

// 3. q/k rms-norm with the baked weights and the gates (beta, log decay), per
// (token, hk).
// grid (T, Hk), block 256: threads 0..127 q, 128..255 k.
template <int R>
__global__ __launch_bounds__(256) void prefill_prep_kernel(
    int Hk, int D, const uint16_t* __restrict__ xc, const uint16_t* __restrict__ ab,
    const float* __restrict__ A_log, const float* __restrict__ dt_bias,
    uint16_t* __restrict__ qn, uint16_t* __restrict__ kn, uint16_t* __restrict__ beta,
    float* __restrict__ lg) {
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
    // log of the decay multiplier g = exp(lg) (compiled_ops.rs:36-43); the
    // naive softplus overflows to inf for a+dt_bias >~ 88 (g = 0), clamped so
    // that differences of cumulative sums stay finite (exp(-1e4) == 0 in f32)
    const float sp = logf(expf(araw + dt_bias[h]) + 1.0f);
    lg[(size_t)t * Hv + h] = fmaxf(-(expf(A_log[h]) * sp), -1.0e4f);
  }
}

// 4. Chunked (WY form) recurrence, one work-group of 256 threads per
// (sequence, value head, 64-row block of Dv), walking the sequence's chunks
// of kC = 64 tokens. With G the cumulative log decay inside a chunk, the
// chunk start state S ([Dv, Dk]) and T = (I + L)^-1,
//   L_ij = beta_i (k_i.k_j) exp(G_i - G_j)   (j < i)
//   P_ij = (q_i.k_j) exp(G_i - G_j)          (j <= i)
//   R    = beta * (V - exp(G) * (K S^T))      per token row
//   V'   = T R
//   O    = exp(G) * (Q S^T) + P V'
//   S^T <- exp(G_C) S^T + K^T (exp(G_C - G) * V')
// which equals the token-by-token recurrence of metal_gdn.rs:37-62.
// Products use v_mfma_f32_16x16x32_bf16: k and q are bf16 already (exact);
// f32 operands on the state path (S, T, R, V') are split into bf16 hi + lo
// parts so they carry ~16 mantissa bits. The state lives in MFMA
// accumulators (S^T tiles) across chunks, with an f32 copy in LDS as the B
// operand of K S^T and Q S^T. Padded rows of a partial chunk have k = q =
// v = beta = 0 and log decay 0, so they leave every result unchanged.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

namespace {
constexpr int kC = 64;
constexpr int kDVB = 64;
constexpr int kLdK = kDk + 8;   // bf16 [64][128] rows (272 B)
constexpr int kLdT = kC + 8;    // bf16 [*][64] rows (144 B)
constexpr int kLdF = kC + 4;    // f32 [*][64] rows (272 B)
constexpr int kLdS = kDk + 4;   // f32 [64][128] rows (528 B)

struct ChunkSmem {
  uint16_t K[kC][kLdK];    // k, token-major
  uint16_t KT[kDk][kLdT];  // k, dk-major
  uint16_t Q[kC][kLdK];    // q, token-major
  uint16_t V[kC][kLdT];    // v of this Dv block, token-major
  uint16_t P[kC][kLdT];    // masked, decayed q.k
  float Tm[kC][kLdF];      // L, then T = (I + L)^-1
  float RV[kDVB][kLdF];    // R^T, then V'^T ([dv][token])
  float S[kDVB][kLdS];     // state block [dv][dk] (chunk start)
  float X[4][16][16];      // per-wave block scratch of the solve
  float beta[kC], G[kC], eG[kC], dec_end[kC];
};

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Operand fragment of a 16x32 (rows x k) block whose k runs contiguous in
// memory: lane l takes row r0 + l%16, k = k0 + 8*(l/16) .. +7. It serves as
// the A operand (rows = output rows) and as the B operand (rows = output
// columns) of v_mfma_f32_16x16x32_bf16.
__device__ __forceinline__ bf16x8 frag(const uint16_t* base, int ld, int r0, int k0, int lane) {
  return *reinterpret_cast<const bf16x8*>(base + (r0 + (lane & 15)) * ld + k0 + (lane >> 4) * 8);
}

__device__ __forceinline__ void split8(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const __bf16 h = (__bf16)x[u];
    hi[u] = h;
    lo[u] = (__bf16)(x[u] - (float)h);
  }
}

// The same fragment taken from f32 storage and split into hi + lo; `scale`
// (indexed by k) multiplies the values first when given.
__device__ __forceinline__ void frag_split(const float* base, int ld, int r0, int k0, int lane,
                                           const float* scale, bf16x8& hi, bf16x8& lo) {
  const int k = k0 + (lane >> 4) * 8;
  const float* p = base + (r0 + (lane & 15)) * ld + k;
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  float x[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  if (scale) {
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] *= scale[k + u];
  }
  split8(x, hi, lo);
}
}  // namespace

template <int R>
__global__ __launch_bounds__(256) void prefill_chunk_kernel(
    float* __restrict__ state, const int32_t* __restrict__ slot_ids,
    const int32_t* __restrict__ cu, int num_slots, int Hk, int D, int T,
    const uint16_t* __restrict__ qn, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ xc, const float* __restrict__ lgv,
    const uint16_t* __restrict__ betav, uint16_t* __restrict__ y, uint32_t* __restrict__ status) {
  __shared__ ChunkSmem sm;
  const int dvb = blockIdx.x, hv = blockIdx.y, s = blockIdx.z;
  const int Hv = Hk * R, hk = hv / R;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int slot = slot_ids[s];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0 && dvb == 0 && hv == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
  const int st = min(max(cu[s], 0), T), en = min(max(cu[s + 1], st), T);
  if (en <= st) return;
  const int dv0 = dvb * kDVB;
  float* gstate = state + ((size_t)slot * Hv + hv) * kTileElems;  // [Dv][Dk]
  const int lr = (lane >> 4) * 4, lc = lane & 15;  // accumulator row base / column

  // state accumulators: S^T tiles, dk block 2*wave + a, dv block J
  f32x4 acc[2][4];
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const int dk = 16 * (2 * wave + a) + lr, dv = 16 * J + lc;
      acc[a][J] = *reinterpret_cast<const f32x4*>(gstate + (size_t)(dv0 + dv) * kDk + dk);
      *reinterpret_cast<f32x4*>(&sm.S[dv][dk]) = acc[a][J];
    }

  const size_t vcol = 2 * (size_t)Hk * kDk + (size_t)hv * kDv + dv0;
  for (int c0 = st; c0 < en; c0 += kC) {
    const int n = min(kC, en - c0);
    // (a) chunk inputs -> LDS; rows >= n are zero
    {
      uint4 kv[4], qv[4], vv[2];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, i = e >> 4, c = (e & 15) * 8;
        kv[u] = make_uint4(0u, 0u, 0u, 0u);
        qv[u] = kv[u];
        if (i < n) {
          const size_t off = ((size_t)(c0 + i) * Hk + hk) * kDk + c;
          kv[u] = *reinterpret_cast<const uint4*>(kn + off);
          qv[u] = *reinterpret_cast<const uint4*>(qn + off);
        }
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = tid + 256 * u, i = e >> 3, c = (e & 7) * 8;
        vv[u] = make_uint4(0u, 0u, 0u, 0u);
        if (i < n) vv[u] = *reinterpret_cast<const uint4*>(xc + (size_t)(c0 + i) * D + vcol + c);
      }
      float b = 0.f, l = 0.f;
      if (wave == 0 && lane < n) {
        b = bf2f(betav[(size_t)(c0 + lane) * Hv + hv]);
        l = lgv[(size_t)(c0 + lane) * Hv + hv];
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int e = tid + 256 * u, i = e >> 4, c = (e & 15) * 8;
        *reinterpret_cast<uint4*>(&sm.K[i][c]) = kv[u];
        *reinterpret_cast<uint4*>(&sm.Q[i][c]) = qv[u];
        const uint16_t* kb = reinterpret_cast<const uint16_t*>(&kv[u]);
#pragma unroll
        for (int w = 0; w < 8; ++w) sm.KT[c + w][i] = kb[w];
      }
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int e = tid + 256 * u, i = e >> 3, c = (e & 7) * 8;
        *reinterpret_cast<uint4*>(&sm.V[i][c]) = vv[u];
      }
      if (wave == 0) {  // inclusive prefix sum of the log decay
        float gsum = l;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const float t = __shfl_up(gsum, off, 64);
          if (lane >= off) gsum += t;
        }
        const float gC = __shfl(gsum, 63, 64);
        sm.beta[lane] = b;
        sm.G[lane] = gsum;
        sm.eG[lane] = expf(gsum);
        sm.dec_end[lane] = expf(gC - gsum);
      }
    }
    __syncthreads();

    // (b) K K^T, Q K^T -> L (Tm, f32) and P (bf16); wave owns row block `wave`
    {
      f32x4 akk[4], aqk[4];
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        akk[J] = f32x4{0.f, 0.f, 0.f, 0.f};
        aqk[J] = akk[J];
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 ak = frag(&sm.K[0][0], kLdK, 16 * wave, 32 * ks, lane);
        const bf16x8 aq = frag(&sm.Q[0][0], kLdK, 16 * wave, 32 * ks, lane);
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          const bf16x8 bk = frag(&sm.K[0][0], kLdK, 16 * J, 32 * ks, lane);
          akk[J] = mfma16(ak, bk, akk[J]);
          aqk[J] = mfma16(aq, bk, aqk[J]);
        }
      }
#pragma unroll
      for (int J = 0; J < 4; ++J)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * wave + lr + r, j = 16 * J + lc;
          const float d = expf(fminf(sm.G[i] - sm.G[j], 0.f));
          sm.Tm[i][j] = j < i ? sm.beta[i] * akk[J][r] * d : 0.f;
          sm.P[i][j] = f2bf(j <= i ? aqk[J][r] * d : 0.f);
        }
    }

    // (d) K S^T and Q S^T for this wave's token rows (independent of (c))
    f32x4 yk[4], zq[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      yk[J] = f32x4{0.f, 0.f, 0.f, 0.f};
      zq[J] = yk[J];
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 ak = frag(&sm.K[0][0], kLdK, 16 * wave, 32 * ks, lane);
      const bf16x8 aq = frag(&sm.Q[0][0], kLdK, 16 * wave, 32 * ks, lane);
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        bf16x8 sh, sl;
        frag_split(&sm.S[0][0], kLdS, 16 * J, 32 * ks, lane, nullptr, sh, sl);
        yk[J] = mfma16(ak, sh, yk[J]);
        yk[J] = mfma16(ak, sl, yk[J]);
        zq[J] = mfma16(aq, sh, zq[J]);
        zq[J] = mfma16(aq, sl, zq[J]);
      }
    }
    __syncthreads();

    // (c) T = (I + L)^-1 in place: 16x16 diagonal blocks by forward
    // substitution (wave b, lanes = columns), then block rows 1..3 with
    // T_ij = -D_i sum_{k=j}^{i-1} L_ik T_kj (all X_ij read L before any T_ij
    // overwrites it).
    if (lane < 16) {
      const int b0 = 16 * wave, j = lane;
      float t[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float a = i == j ? 1.f : 0.f;
#pragma unroll
        for (int k = 0; k < i; ++k) a -= sm.Tm[b0 + i][b0 + k] * t[k];
        t[i] = a;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) sm.Tm[b0 + i][b0 + j] = t[i];
    }
    __syncthreads();
    {
      const int rr = lane >> 2, cq = (lane & 3) * 4;
      for (int bi = 1; bi < 4; ++bi) {
        if (wave < bi) {
          f32x4 x = {0.f, 0.f, 0.f, 0.f};
          for (int kb = wave; kb < bi; ++kb)
#pragma unroll
            for (int m = 0; m < 16; ++m)
              x += sm.Tm[16 * bi + rr][16 * kb + m] *
                   *reinterpret_cast<const f32x4*>(&sm.Tm[16 * kb + m][16 * wave + cq]);
          *reinterpret_cast<f32x4*>(&sm.X[wave][rr][cq]) = x;
        }
        __syncthreads();
        if (wave < bi) {
          f32x4 t = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int m = 0; m < 16; ++m)
            t += sm.Tm[16 * bi + rr][16 * bi + m] *
                 *reinterpret_cast<const f32x4*>(&sm.X[wave][m][cq]);
          *reinterpret_cast<f32x4*>(&sm.Tm[16 * bi + rr][16 * wave + cq]) = -t;
        }
        __syncthreads();
      }
    }

    // (e) R = beta * (V - exp(G) * K S^T), stored transposed [dv][token]
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * wave + lr + r, dv = 16 * J + lc;
        sm.RV[dv][i] = sm.beta[i] * (bf2f(sm.V[i][dv]) - sm.eG[i] * yk[J][r]);
      }
    __syncthreads();

    // (f) V' = T R (T lower triangular: k blocks above the row block are 0)
    f32x4 vp[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) vp[J] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (32 * ks > 16 * wave + 15) continue;
      bf16x8 th, tl;
      frag_split(&sm.Tm[0][0], kLdF, 16 * wave, 32 * ks, lane, nullptr, th, tl);
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        bf16x8 rh, rl;
        frag_split(&sm.RV[0][0], kLdF, 16 * J, 32 * ks, lane, nullptr, rh, rl);
        vp[J] = mfma16(th, rh, vp[J]);
        vp[J] = mfma16(th, rl, vp[J]);
        vp[J] = mfma16(tl, rh, vp[J]);
      }
    }
    __syncthreads();
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int r = 0; r < 4; ++r) sm.RV[16 * J + lc][16 * wave + lr + r] = vp[J][r];
    __syncthreads();

    // (g) O = exp(G) * Q S^T + P V'
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int r = 0; r < 4; ++r) zq[J][r] *= sm.eG[16 * wave + lr + r];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if (32 * ks > 16 * wave + 15) continue;
      const bf16x8 ap = frag(&sm.P[0][0], kLdT, 16 * wave, 32 * ks, lane);
#pragma unroll
      for (int J = 0; J < 4; ++J) {
        bf16x8 vh, vl;
        frag_split(&sm.RV[0][0], kLdF, 16 * J, 32 * ks, lane, nullptr, vh, vl);
        zq[J] = mfma16(ap, vh, zq[J]);
        zq[J] = mfma16(ap, vl, zq[J]);
      }
    }
#pragma unroll
    for (int J = 0; J < 4; ++J)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * wave + lr + r;
        if (i < n) y[((size_t)(c0 + i) * Hv + hv) * kDv + dv0 + 16 * J + lc] = f2bf(zq[J][r]);
      }

    // (h) S^T <- exp(G_C) S^T + K^T (exp(G_C - G) * V')
    const float eC = sm.eG[kC - 1];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int J = 0; J < 4; ++J) acc[a][J] *= eC;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const bf16x8 ak = frag(&sm.KT[0][0], kLdT, 16 * (2 * wave + a), 32 * ks, lane);
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          bf16x8 vh, vl;
          frag_split(&sm.RV[0][0], kLdF, 16 * J, 32 * ks, lane, sm.dec_end, vh, vl);
          acc[a][J] = mfma16(ak, vh, acc[a][J]);
          acc[a][J] = mfma16(ak, vl, acc[a][J]);
        }
      }
    }
    __syncthreads();
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int J = 0; J < 4; ++J)
        *reinterpret_cast<f32x4*>(&sm.S[16 * J + lc][16 * (2 * wave + a) + lr]) = acc[a][J];
    __syncthreads();
  }
#pragma unroll
  for (int a = 0; a < 2; ++a)
#pragma unroll
    for (int J = 0; J < 4; ++J)
      *reinterpret_cast<f32x4*>(gstate + (size_t)(dv0 + 16 * J + lc) * kDk + 16 * (2 * wave + a) +
                                lr) = acc[a][J];
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
                       ws.beta, ws.lg);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(prefill_chunk_kernel<R>, dim3(kDv / kDVB, Hv, a.nseq), dim3(256), 0,
                     a.stream, a.state, a.slot_ids, a.cu_seqlens, a.num_slots, a.Hk, D,
                     a.total_tokens, ws.qn, ws.kn, ws.xc, ws.lg, ws.beta, a.y, a.status);
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
