// gdn_qlinear.hip -- the 4-bit affine-quantized linear layer that produces the
// GDN block's merged input projections on gfx950:
//   qkvz = quantized_matmul(x, W_qkv|W_z, ..., transpose, group 64, bits 4)
//   ab   = quantized_matmul(x, W_b|W_a,   ...)            (qwen3_5.rs:572-586)
// with the parts concatenated along the output axis once, at load time, as the
// reference merges them (qwen3_5.rs:1037-1053).
//
// Source format (MLX affine quantization, mlx-rs 0.25.3 / mlx-sys 0.2.0):
//   W uint32 [N, K/8]: element k of row n is the nibble q at bits 4*(k%8) of
//   word k/8; scales s, biases b bf16 [N, K/64]; w[n,k] = s[n,k/64]*q + b[n,k/64].
//
// Arithmetic. With groups g of 64 k and X_g[m] = sum_{k in g} x[m,k]:
//   y[m,n] = sum_g s[n,g] * sum_{k in g} x[m,k] q[n,k] + sum_g b[n,g] X_g[m].
// The nibbles enter v_mfma_f32_16x16x32_bf16 as the bf16 numbers 128+q (bit
// pattern 0x4300|q; four dwords of two such values come out of one packed
// dword with one v_and_or_b32 each), so the per-group MFMA sum is
// A_g = 128 X_g + sum x q, exact products accumulated in f32, and
//   y = sum_g s_g A_g + sum_g (b_g - 128 s_g) X_g.
// The first sum costs one FMA per output and group. X_g comes from the same
// MFMA against an all-ones operand. The second sum is a short MFMA product at
// the end, X_g split exactly into three bf16 parts (hi + mid + lo) against
// b and -128 s, both exact in bf16. The one rounding to bf16 is the store.
#include "gdn_common.h"

namespace gdn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kStageK = 128;    // k per pipeline stage: two groups
constexpr int kMaxGroups = 64;  // K <= 4096
constexpr int kWideDecodeN = 131072;  // decode-sized calls at least this wide use 64 x 128 tiles

__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// One packed dword (nibble order k0 k2 k4 k6 k1 k3 k5 k7 of eight consecutive
// k) -> the MFMA operand dwords (128+q_k0, 128+q_k1), ..., (128+q_k6, 128+q_k7).
// m = 0x000F000F held in a VGPR: with one literal left, (v & m) | e selects a
// single v_and_or_b32 (gfx950 VOP3 takes no literal, the exponent bits go in
// an SGPR); with both constants literal the compiler emits v_and + v_or.
// (Written in C, not inline asm: the hazard recognizer cannot see into inline
// asm, and a VALU write into a VGPR an in-flight MFMA still reads as its
// accumulator input needs wait states it then does not insert.)
__device__ __forceinline__ u32x4 unpack_w(uint32_t w, uint32_t m) {
  const uint32_t e = 0x43004300u;
  return (u32x4){(w & m) | e, ((w >> 4) & m) | e, ((w >> 8) & m) | e, ((w >> 12) & m) | e};
}

// Packed layout written by qlinear_pack_kernel, per 16-row fragment f and
// k-pair p (128 k, two groups):
//   weights  wp[(f*P + p)*64 + lane]   u32x4, lane = 16c + r (row r of the
//            fragment, k-block c): dword 2*gl + h covers the eight k
//            128p + 64gl + 32h + 8c + (0..7) in the nibble order above;
//   scales   sp[((f*P + p)*16 + r)*2 + gl]  bf16;
//   biases   bias[n*G + g], and nsc[n*G + g] = -128 * s[n,g], bf16 (exact).
__global__ void qlinear_pack_kernel(const uint32_t* __restrict__ w, const uint16_t* __restrict__ s,
                                    const uint16_t* __restrict__ b, int N, int K, int frag0,
                                    u32x4* __restrict__ wp, uint16_t* __restrict__ sp,
                                    uint16_t* __restrict__ bias, uint16_t* __restrict__ nsc) {
  const int P = K >> 7, G = K >> 6, words = K >> 3;
  const int64_t total = (int64_t)(N >> 4) * P * 64;
  for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
       t += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(t & 63);
    const int64_t fp = t >> 6;
    const int p = (int)(fp % P), f = (int)(fp / P);
    const int r = lane & 15, c = lane >> 4, n = f * 16 + r;
    u32x4 o;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int gl = j >> 1, h = j & 1;
      const uint32_t v = w[(int64_t)n * words + 16 * p + 8 * gl + 4 * h + c];
      uint32_t q = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        q |= ((v >> (8 * i)) & 0xFu) << (4 * i);            // k = 2i     -> nibble i
        q |= ((v >> (8 * i + 4)) & 0xFu) << (4 * (i + 4));  // k = 2i + 1 -> nibble i+4
      }
      o[j] = q;
    }
    const int64_t fd = (int64_t)(frag0 + f) * P + p;
    wp[fd * 64 + lane] = o;
    if (lane < 32) {
      const int rr = lane >> 1, gl = lane & 1;
      sp[(fd * 16 + rr) * 2 + gl] = s[(int64_t)(f * 16 + rr) * G + 2 * p + gl];
    }
    if (lane < 2) {  // biases and -128*scales of row n, groups 2p, 2p+1
      const int r0 = (frag0 + f) * 16;
      for (int rr = 0; rr < 16; ++rr) {
        const int64_t src = (int64_t)(f * 16 + rr) * G + 2 * p + lane;
        const int64_t dst = (int64_t)(r0 + rr) * G + 2 * p + lane;
        bias[dst] = b[src];
        nsc[dst] = f2bf(-128.0f * bf2f(s[src]));
      }
    }
  }
}

// y[m, n] for a work-group tile of MT = 16*MW*WM rows (m) by NT = 16*NW*WN
// columns (n); wave (wm, wn) owns MW row fragments and NW column fragments.
// The weight fragment is the MFMA A operand (16 n x 32 k), the activation
// fragment the B operand (32 k x 16 m), so each lane ends with four
// consecutive n of one row m: D[4c + r][m], c = lane/16.
// x is staged through LDS in stages of 128 k (double buffered, rows of 256 B
// with the 16-byte chunk index XOR-swizzled by row so fragment reads are
// conflict-free); weights and scales go straight from global memory to
// registers one stage ahead.
template <int MW, int NW, int WM, int WN>
__global__ __launch_bounds__(256) void qlinear_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, int K, const u32x4* __restrict__ wp,
    const uint16_t* __restrict__ sp, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ nsc, int N, uint16_t* __restrict__ y, int64_t ys) {
  static_assert(WM * WN == 4, "four waves per work-group");
  constexpr int MT = 16 * MW * WM, NT = 16 * NW * WN;
  constexpr int XROW = kStageK * 2;  // bytes per staged x row
  constexpr int SJ = MT / 16;        // staged uint4 per thread per stage
  __shared__ __align__(16) uint8_t xl[2][MT * XROW];
  __shared__ float sx[kMaxGroups * MT];  // X_g[m] at sx[g*MT + m]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int G = K >> 6, P = K >> 7;
  const int m0 = blockIdx.y * MT;
  const int f0 = blockIdx.x * (NT / 16) + wn * NW;  // first column fragment of the wave
  const int r16 = lane & 15, c4 = lane >> 4;

  // staging: thread -> rows srow + 16j, 16-byte chunk sch
  const int srow = tid >> 4, sch = tid & 15;
  const int sdst = srow * XROW + ((sch ^ (srow & 15)) << 4);
  const uint16_t* xsrc[SJ];
#pragma unroll
  for (int j = 0; j < SJ; ++j) {
    const int r = min(m0 + srow + 16 * j, M - 1);
    xsrc[j] = x + (int64_t)r * xs + sch * 8;
  }
  u32x4 stg[SJ];
  const u32x4* wsrc[NW];
  const u32x4* ssrc[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    wsrc[i] = wp + (int64_t)(f0 + i) * P * 64 + lane;
    ssrc[i] = reinterpret_cast<const u32x4*>(sp) + (int64_t)(f0 + i) * P * 4 + c4;
  }

  u32x4 wc[NW], sc[NW], wnx[NW], snx[NW];
#pragma unroll
  for (int j = 0; j < SJ; ++j) stg[j] = *reinterpret_cast<const u32x4*>(xsrc[j]);
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    wc[i] = wsrc[i][0];
    sc[i] = ssrc[i][0];
  }
#pragma unroll
  for (int j = 0; j < SJ; ++j) *reinterpret_cast<u32x4*>(&xl[0][sdst + 16 * j * XROW]) = stg[j];
  lds_barrier();

  f32x4 T[NW][MW];
#pragma unroll
  for (int i = 0; i < NW; ++i)
#pragma unroll
    for (int u = 0; u < MW; ++u) T[i][u] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  uint32_t nib = 0x000F000Fu;
  asm volatile("" : "+v"(nib));  // keep the nibble mask in a VGPR

  // Straight-line stage body: the last stage reloads itself and writes the
  // idle LDS buffer instead of branching (a branch around the prefetch made
  // the compiler keep more registers live and cost 5%).
  for (int p = 0; p < P; ++p) {
    const int buf = p & 1;
    const int pn = min(p + 1, P - 1);
    {
#pragma unroll
      for (int j = 0; j < SJ; ++j)
        stg[j] = *reinterpret_cast<const u32x4*>(xsrc[j] + pn * kStageK);
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        wnx[i] = wsrc[i][pn * 64];
        snx[i] = ssrc[i][pn * 4];
      }
    }
#pragma unroll
    for (int gl = 0; gl < 2; ++gl) {
      u32x4 X[MW][2];
#pragma unroll
      for (int u = 0; u < MW; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = (wm * MW + u) * 16 + r16;
          const int ch = 8 * gl + 4 * h + c4;
          X[u][h] = *reinterpret_cast<const u32x4*>(&xl[buf][row * XROW + ((ch ^ r16) << 4)]);
        }
      // X_g of the row fragments this wave owns (u % WN == wn)
#pragma unroll
      for (int u = 0; u < MW; ++u)
        if (u % WN == wn) {
          f32x4 a = mfma(ones, X[u][0], zero);
          a = mfma(ones, X[u][1], a);
          sx[(2 * p + gl) * MT + (wm * MW + u) * 16 + r16] = a[0];  // the 4 lane groups agree
        }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const u32x4 A0 = unpack_w(wc[i][2 * gl], nib), A1 = unpack_w(wc[i][2 * gl + 1], nib);
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = gl ? bf_hi(sc[i][r]) : bf_lo(sc[i][r]);
#pragma unroll
        for (int u = 0; u < MW; ++u) {
          f32x4 a = mfma(A0, X[u][0], zero);
          a = mfma(A1, X[u][1], a);
#pragma unroll
          for (int r = 0; r < 4; ++r) T[i][u][r] = fmaf(s[r], a[r], T[i][u][r]);
        }
      }
    }
    {
#pragma unroll
      for (int j = 0; j < SJ; ++j)
        *reinterpret_cast<u32x4*>(&xl[buf ^ 1][sdst + 16 * j * XROW]) = stg[j];
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        wc[i] = wnx[i];
        sc[i] = snx[i];
      }
    }
    lds_barrier();
  }

  // sum_g (b_g - 128 s_g) X_g, X_g = hi + mid + lo exactly
  for (int j = 0; j < G; j += 32) {
    const bool gin = j + 8 * c4 < G;  // G is a multiple of 8
#pragma unroll
    for (int u = 0; u < MW; ++u) {
      const int row = (wm * MW + u) * 16 + r16;
      u32x4 hi, mid, lo;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float v0 = 0.f, v1 = 0.f;
        if (gin) {
          v0 = sx[(j + 8 * c4 + e) * MT + row];
          v1 = sx[(j + 8 * c4 + e + 1) * MT + row];
        }
        const uint32_t h = f2bf2(v0, v1);
        const float r0 = v0 - bf_lo(h), r1 = v1 - bf_hi(h);
        const uint32_t md = f2bf2(r0, r1);
        hi[e >> 1] = h;
        mid[e >> 1] = md;
        lo[e >> 1] = f2bf2(r0 - bf_lo(md), r1 - bf_hi(md));
      }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const int64_t n = (int64_t)(f0 + i) * 16 + r16;
        u32x4 Ab = {0u, 0u, 0u, 0u}, As = {0u, 0u, 0u, 0u};
        if (gin) {
          Ab = *reinterpret_cast<const u32x4*>(bias + n * G + j + 8 * c4);
          As = *reinterpret_cast<const u32x4*>(nsc + n * G + j + 8 * c4);
        }
        f32x4 t = T[i][u];
        t = mfma(Ab, hi, t);
        t = mfma(Ab, mid, t);
        t = mfma(Ab, lo, t);
        t = mfma(As, hi, t);
        t = mfma(As, mid, t);
        t = mfma(As, lo, t);
        T[i][u] = t;
      }
    }
  }

#pragma unroll
  for (int u = 0; u < MW; ++u) {
    const int m = m0 + (wm * MW + u) * 16 + r16;
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const int n = (f0 + i) * 16 + 4 * c4;
      if (m < M && n < N) {
        const f32x4 t = T[i][u];
        *reinterpret_cast<u32x2*>(y + (int64_t)m * ys + n) = (u32x2){f2bf2(t[0], t[1]), f2bf2(t[2], t[3])};
      }
    }
  }
}

// Decode shapes (M <= 64): one 64-row tile, 64 columns per work-group, the K
// axis split over KS groups of four waves (wave w: column fragment w % 4, K
// part w / 4) that add their sums through LDS at the end. A launch of a few
// hundred work-groups with one column fragment per wave is latency-bound, so
// the S stages of a K part are unrolled and every load is issued early in
// stage order: x of the first three stages, then the wave's whole weight and
// scale slice and its correction operands, then x three stages ahead of use.
// Vector-memory counters drain in issue order, so each stage waits only for
// its own weights and x, never for the loads queued behind them.
//
// A work-group covers the K slice [kof, kof + 128 KS S) of a K-wide layer,
// kof = 128 KS S * blockIdx.y. With one slice (gridDim.y == 1) it writes bf16
// y; with several (layers too narrow in N to fill the chip) it writes its f32
// partial sums, correction of its own groups included, to
// part[blockIdx.y][m][n] (row stride Npad), and qlinear_sum_kernel adds the
// slices in order and rounds once.
template <int KS, int S>
__global__ __launch_bounds__(256 * KS) void qlinear_decode_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, int K, const u32x4* __restrict__ wp,
    const uint16_t* __restrict__ sp, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ nsc, int N, uint16_t* __restrict__ y, int64_t ys,
    float* __restrict__ part, int Npad) {
  static_assert(S >= 2 && S % 2 == 0, "S stages per K part, alternating x buffers");
  constexpr int MT = 64, XROW = kStageK * 2, SJ = MT / 16;
  constexpr int G = 2 * KS * S;  // groups of the work-group's K slice
  __shared__ __align__(16) uint8_t xl[KS][2][MT * XROW];
  __shared__ float sx[G * MT];  // X_g[m] at sx[g*MT + m], g local to the slice

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ks = wave >> 2, wn = wave & 3;
  const int Ptot = K >> 7, Gtot = K >> 6;
  const int pbase = blockIdx.y * (KS * S);  // first stage of the slice in the layer
  const int p0 = ks * S;                    // first stage of the wave's K part in the slice
  const int f = blockIdx.x * 4 + wn;  // the wave's column fragment
  const int r16 = lane & 15, c4 = lane >> 4;

  // x staging: thread -> rows srow + 16j, chunk sch, of this K part
  const int lt = tid & 255, srow = lt >> 4, sch = lt & 15;
  const int sdst = srow * XROW + ((sch ^ srow) << 4);
  const uint16_t* xsrc[SJ];
#pragma unroll
  for (int j = 0; j < SJ; ++j)
    xsrc[j] = x + (int64_t)min(srow + 16 * j, M - 1) * xs + sch * 8 + (pbase + p0) * kStageK;
  constexpr int XD = S < 3 ? S : 3;  // x stages in flight
  u32x4 R[XD][SJ];
#pragma unroll
  for (int q = 0; q < XD; ++q) {
#pragma unroll
    for (int j = 0; j < SJ; ++j) R[q][j] = *reinterpret_cast<const u32x4*>(xsrc[j] + q * kStageK);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order (the counters drain in it)
  }

  // Weights, scales and the correction operands are read once: nontemporal,
  // so the stream does not evict x, which every work-group re-reads, from L2.
  const u32x4* wsrc = wp + ((int64_t)f * Ptot + pbase + p0) * 64 + lane;
  const u32x4* ssrc = reinterpret_cast<const u32x4*>(sp) + ((int64_t)f * Ptot + pbase + p0) * 4 + c4;
  u32x4 wr[S], sr[S];
#pragma unroll
  for (int p = 0; p < S; ++p) {
    wr[p] = __builtin_nontemporal_load(wsrc + p * 64);
    sr[p] = __builtin_nontemporal_load(ssrc + p * 4);
    __builtin_amdgcn_sched_barrier(0);
  }
  constexpr int GJ = (G + 31) / 32;  // 32-group blocks of the correction
  u32x4 Ab[GJ], As[GJ];
#pragma unroll
  for (int j = 0; j < GJ; ++j) {
    Ab[j] = As[j] = (u32x4){0u, 0u, 0u, 0u};
    if (32 * j + 8 * c4 < G) {  // G is a multiple of 8: whole 8-group words
      const int64_t o = ((int64_t)f * 16 + r16) * Gtot + 2 * pbase + 32 * j + 8 * c4;
      Ab[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bias + o));
      As[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nsc + o));
    }
  }
  __builtin_amdgcn_sched_barrier(0);

#pragma unroll
  for (int j = 0; j < SJ; ++j) *reinterpret_cast<u32x4*>(&xl[ks][0][sdst + 16 * j * XROW]) = R[0][j];
  lds_barrier();

  f32x4 T[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) T[u] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  uint32_t nib = 0x000F000Fu;
  asm volatile("" : "+v"(nib));

#pragma unroll
  for (int p = 0; p < S; ++p) {
    const int b = p & 1;
    if (p + XD < S) {  // x of stage p+XD into the registers stage p's x came in
#pragma unroll
      for (int i = 0; i < SJ; ++i)
        R[p % XD][i] = *reinterpret_cast<const u32x4*>(xsrc[i] + (p + XD) * kStageK);
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* xb = xl[ks][b];
#pragma unroll
    for (int gl = 0; gl < 2; ++gl) {
      u32x4 X[4][2];
#pragma unroll
      for (int u = 0; u < 4; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int ch = 8 * gl + 4 * h + c4;
          X[u][h] = *reinterpret_cast<const u32x4*>(&xb[(u * 16 + r16) * XROW + ((ch ^ r16) << 4)]);
        }
      {  // X_g of row fragment wn
        const int row = wn * 16 + r16;
        const u32x4 s0 = *reinterpret_cast<const u32x4*>(&xb[row * XROW + (((8 * gl + c4) ^ r16) << 4)]);
        const u32x4 s1 = *reinterpret_cast<const u32x4*>(&xb[row * XROW + (((8 * gl + 4 + c4) ^ r16) << 4)]);
        f32x4 a = mfma(ones, s0, zero);
        a = mfma(ones, s1, a);
        if (c4 == 0) sx[(2 * (p0 + p) + gl) * MT + row] = a[0];
      }
      const u32x4 A0 = unpack_w(wr[p][2 * gl], nib), A1 = unpack_w(wr[p][2 * gl + 1], nib);
      float sc[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) sc[r] = gl ? bf_hi(sr[p][r]) : bf_lo(sr[p][r]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f32x4 a = mfma(A0, X[u][0], zero);
        a = mfma(A1, X[u][1], a);
#pragma unroll
        for (int r = 0; r < 4; ++r) T[u][r] = fmaf(sc[r], a[r], T[u][r]);
      }
    }
    if (p + 1 < S) {  // x of stage p+1 into the other buffer (last read in stage p-1)
#pragma unroll
      for (int i = 0; i < SJ; ++i)
        *reinterpret_cast<u32x4*>(&xl[ks][b ^ 1][sdst + 16 * i * XROW]) = R[(p + 1) % XD][i];
    }
    lds_barrier();
  }

  if (KS > 1) {  // K parts 1.. hand their sums to part 0 through the (now idle) x buffers
    f32x4* red = reinterpret_cast<f32x4*>(&xl[0][0][0]);
    if (ks > 0) {
#pragma unroll
      for (int u = 0; u < 4; ++u) red[(((ks - 1) * 4 + wn) * 4 + u) * 64 + lane] = T[u];
    }
    lds_barrier();
    if (ks > 0) return;
    for (int k2 = 1; k2 < KS; ++k2)
#pragma unroll
      for (int u = 0; u < 4; ++u) T[u] += red[(((k2 - 1) * 4 + wn) * 4 + u) * 64 + lane];
  }

  // sum_g (b_g - 128 s_g) X_g with X_g = hi + mid + lo
#pragma unroll
  for (int jb = 0; jb < GJ; ++jb) {
    const int j = 32 * jb;
    const bool gin = j + 8 * c4 < G;
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int row = u * 16 + r16;
      u32x4 hi, mid, lo;
#pragma unroll
      for (int e = 0; e < 8; e += 2) {
        float v0 = 0.f, v1 = 0.f;
        if (gin) {
          v0 = sx[(j + 8 * c4 + e) * MT + row];
          v1 = sx[(j + 8 * c4 + e + 1) * MT + row];
        }
        const uint32_t h = f2bf2(v0, v1);
        const float q0 = v0 - bf_lo(h), q1 = v1 - bf_hi(h);
        const uint32_t md = f2bf2(q0, q1);
        hi[e >> 1] = h;
        mid[e >> 1] = md;
        lo[e >> 1] = f2bf2(q0 - bf_lo(md), q1 - bf_hi(md));
      }
      f32x4 t = T[u];
      t = mfma(Ab[jb], hi, t);
      t = mfma(Ab[jb], mid, t);
      t = mfma(Ab[jb], lo, t);
      t = mfma(As[jb], hi, t);
      t = mfma(As[jb], mid, t);
      t = mfma(As[jb], lo, t);
      T[u] = t;
    }
  }

  const int n = f * 16 + 4 * c4;
  if (part != nullptr) {  // f32 partial of this K slice (all Npad columns)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int m = u * 16 + r16;
      if (m < M)
        *reinterpret_cast<f32x4*>(part + ((int64_t)blockIdx.y * MT + m) * Npad + n) = T[u];
    }
  } else if (n < N) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int m = u * 16 + r16;
      if (m < M)
        *reinterpret_cast<u32x2*>(y + (int64_t)m * ys + n) =
            (u32x2){f2bf2(T[u][0], T[u][1]), f2bf2(T[u][2], T[u][3])};
    }
  }
}

// y[m, n..n+3] = bf16(sum over the K slices, in slice order, of the f32
// partials of qlinear_decode_kernel). grid ceil(M * Npad / 4 / 256), block 256.
__global__ __launch_bounds__(256) void qlinear_sum_kernel(const float* __restrict__ part,
                                                          int nslice, int M, int N, int Npad,
                                                          uint16_t* __restrict__ y, int64_t ys) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index in [M, Npad]
  const int q = Npad / 4;
  if (i >= (int64_t)M * q) return;
  const int m = (int)(i / q), n = (int)(i % q) * 4;
  if (n >= N) return;
  f32x4 t = *reinterpret_cast<const f32x4*>(part + (int64_t)m * Npad + n);
  for (int sl = 1; sl < nslice; ++sl)
    t += *reinterpret_cast<const f32x4*>(part + ((int64_t)sl * 64 + m) * Npad + n);
  *reinterpret_cast<u32x2*>(y + (int64_t)m * ys + n) = (u32x2){f2bf2(t[0], t[1]), f2bf2(t[2], t[3])};
}

template <int MW, int NW, int WM, int WN>
hipError_t launch_cfg(const QLinearArgs& a) {
  constexpr int MT = 16 * MW * WM, NT = 16 * NW * WN;
  const dim3 grid(a.Npad / NT, (a.M + MT - 1) / MT);
  hipLaunchKernelGGL((qlinear_kernel<MW, NW, WM, WN>), grid, dim3(256), 0, a.stream, a.x, a.xs,
                     a.M, a.K, reinterpret_cast<const u32x4*>(a.wp), a.sp, a.bias, a.nsc, a.N,
                     a.y, a.ys);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_qlinear_pack(const QLinearPackArgs& a) {
  const int64_t total = (int64_t)(a.N >> 4) * (a.K >> 7) * 64;
  const int64_t want = (total + 255) / 256;
  const int blocks = (int)(want < 4096 ? want : 4096);
  hipLaunchKernelGGL(qlinear_pack_kernel, dim3(blocks), dim3(256), 0, a.stream, a.w, a.s, a.b, a.N,
                     a.K, a.frag0, reinterpret_cast<u32x4*>(a.wp), a.sp, a.bias, a.nsc);
  return hipGetLastError();
}

int qlinear_decode_slices(int K, int Npad) {
  // one work-group per 64 columns; layers with fewer than 128 such groups
  // (out_proj: 2048 columns), and every K above 2048, split K into 512-wide
  // slices (K <= 4096: at most 8); very wide layers take the tiled kernel
  if (K <= 512 || (K <= 2048 && Npad / 64 >= 128) || Npad >= kWideDecodeN) return 1;
  return K / 512;
}

// Tile choice: up to 64 rows (batched decode) qlinear_decode_kernel, whole K
// (K <= 2048) or K slices of 512 (narrow layers, and every K above 2048 --
// those always get a workspace); otherwise 64 x 128 tiles (prefill). Of the
// tilings swept at 16384 x 2048 -> 12352 (four waves each, 16-wide fragments
// per wave m x n: 4x4, 2x4, 4x2, 2x2, 2x4 in one row of waves, 1x4, 2x2 in
// one column), 2 x 4 fragments per wave in a 2 x 2 wave grid was fastest:
// about 200 VGPRs and 48 KB of LDS give two waves per SIMD (1.42 ms; 4 x 4
// with one wave per SIMD took 1.98 ms). Deeper x prefetch (two stages in
// registers) pushed it to one wave per SIMD and 2.06 ms; an XCD-aware tile
// order (each XCD's L2 holding its own weight columns) changed nothing.
//
// Very wide layers at decode sizes (lm_head, 248,320 columns) re-read all of
// x per 64 columns in qlinear_decode_kernel, 4x the weight bytes through L2.
// There a 64 x 128 tile with every wave holding all 64 rows and two column
// fragments (one row of four waves) took 140 us at M = 64, K = 2048, against
// 196 us for the decode kernel, 159 us for the 2 x 2 wave grid and 157 us for
// four column fragments per wave (256 VGPRs, one wave per SIMD).
hipError_t launch_qlinear(const QLinearArgs& a) {
  if (a.defer) *a.defer = QPartial{};
  if (a.M <= 64 && a.Npad >= kWideDecodeN) return launch_cfg<4, 2, 1, 4>(a);
  if (a.M <= 64) {
    const int ns = a.part ? qlinear_decode_slices(a.K, a.Npad) : 1;
    if (ns > 1 || a.K == 512 || a.K == 1024 || a.K == 2048) {
      const u32x4* wp = reinterpret_cast<const u32x4*>(a.wp);
      if (ns > 1) {  // 512-wide slices: two K parts of two stages
        hipLaunchKernelGGL((qlinear_decode_kernel<2, 2>), dim3(a.Npad / 64, ns), dim3(512), 0,
                           a.stream, a.x, a.xs, a.M, a.K, wp, a.sp, a.bias, a.nsc, a.N, a.y, a.ys,
                           a.part, a.Npad);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (a.defer) {  // the consumer adds the slices
          *a.defer = QPartial{a.part, ns, a.Npad};
          return hipSuccess;
        }
        const int64_t n4 = (int64_t)a.M * (a.Npad / 4);
        hipLaunchKernelGGL(qlinear_sum_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                           a.stream, a.part, ns, a.M, a.N, a.Npad, a.y, a.ys);
        return hipGetLastError();
      }
      // two K parts of S = K/256 stages each
      auto kern = a.K == 2048   ? qlinear_decode_kernel<2, 8>
                  : a.K == 1024 ? qlinear_decode_kernel<2, 4>
                                : qlinear_decode_kernel<2, 2>;
      hipLaunchKernelGGL(kern, dim3(a.Npad / 64), dim3(512), 0, a.stream, a.x, a.xs, a.M, a.K, wp,
                         a.sp, a.bias, a.nsc, a.N, a.y, a.ys, nullptr, a.Npad);
      return hipGetLastError();
    }
  }
  return launch_cfg<2, 4, 2, 2>(a);
}

}  // namespace gdn
