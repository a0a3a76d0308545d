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

// s_waitcnt vmcnt(n) (gfx9 encoding; expcnt and lgkmcnt left at their maximum)
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}
__device__ __forceinline__ void wait_lgkm0() { __builtin_amdgcn_s_waitcnt(0xC07F); }

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


// Very wide layers at decode sizes (lm_head): 64 x 128 tiles of four waves in
// a row, every wave with all 64 rows and two 16-column fragments (the weight
// fragment is the MFMA A operand, as in qlinear_kernel). Per stage of 128 k:
//  - x (64 rows x 256 B) is copied into LDS by DMA (buffer_load ... lds: wave
//    w copies rows 4w + 16j .. +3, 1 KiB per load, lane L to byte 16 L of
//    those rows, i.e. physical chunk L % 16 of row 4w + 16j + L / 16, which
//    holds logical chunk (L % 16) ^ (row % 16) -- the swizzle of
//    qlinear_kernel), double buffered;
//  - the weights go to registers one stage ahead;
//  - the scales (64 B per fragment) are copied into LDS by DMA, one 4-byte
//    copy per wave for its two fragments: a 16-byte load per lane of the
//    same block costs the vector memory path as much as a weight load.
// Weights and scales are read through buffer resources with the stage in
// soffset, so no address registers are kept per stage.
// Each stage ends with this wave's copies of the next stage landed (vmcnt 0)
// and a bare barrier: an LDS fence would also count the copies. The ring
// slots are separate arrays, so that the compiler can tell copies into one
// from reads of another.
// Group sums X_g: wave w forms those of its own 16-row block with the
// ones-MFMA and keeps them in registers, lane group c4 holding group 4t + c4
// of ring turn t (a shift register of KT values, KT >= G / 4); they are
// stored to LDS once after the loop. (An LDS store in the loop made the
// compiler wait there for the DMA copies of the next stage.) With XS the
// caller's split sums (xsg [3][64][G] bf16, launch_add_norm's) are copied
// into LDS by DMA with the first stage instead, and no X_g products are
// formed.
// K a multiple of 512 (G a multiple of 8), G <= 4 KT; three waves per SIMD
// for K <= 2048 (KT = 8), two above.
template <int KT, bool XS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(KT <= 8 ? 3 : 2, KT <= 8 ? 3 : 2))) void qlinear_head_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, int K, const uint16_t* __restrict__ wp,
    const uint16_t* __restrict__ sp, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ nsc, int N, int Npad, uint16_t* __restrict__ y, int64_t ys,
    const uint16_t* __restrict__ xsg) {
  constexpr int MW = 4, NW = 2, MT = 64;
  constexpr int XROW = kStageK * 2;  // bytes per staged x row
  constexpr int GMAX = 4 * KT, GJ = GMAX / 32;
  static_assert(GMAX % 32 == 0, "whole 32-group chunks");
  __shared__ __align__(16) uint8_t xl0[MT * XROW];
  __shared__ __align__(16) uint8_t xl1[MT * XROW];
  __shared__ __align__(16) uint8_t sl0[4 * 256];  // per wave: its fragments' 2 x 64 B
  __shared__ __align__(16) uint8_t sl1[4 * 256];
  // X_g: f32 [g][m] (formed here) or the caller's bf16 [3][m][G]
  __shared__ __align__(16) uint8_t sxb[XS ? 3 * MT * GMAX * 2 : GMAX * MT * 4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int G = K >> 6, P = K >> 7;
  const int f0 = blockIdx.x * 8 + wave * NW;  // first column fragment of the wave
  const int r16 = lane & 15, c4 = lane >> 4;

  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)(((int64_t)(M - 1) * xs + K) * 2), 0x00020000);
  const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)wp, (short)0, (int)((int64_t)(Npad / 16) * P * 1024), 0x00020000);
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)sp, (short)0, (int)((int64_t)(Npad / 16) * P * 64), 0x00020000);
  int xvo[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int row = 4 * (wave + 4 * j) + (lane >> 4);
    xvo[j] = (int)((min(row, M - 1) * xs + 8 * ((lane & 15) ^ (row & 15))) * 2);
  }
  const int wvo0 = (f0 * P * 64 + lane) * 16, wvo1 = wvo0 + P * 1024;
  // scale copy: lane L -> fragment f0 + (L % 32) / 16, dword L % 16 (lanes 32-63 repeat 0-31)
  const int svo = ((f0 + ((lane & 31) >> 4)) * P * 64 + 4 * (lane & 15));

  u32x4 w0[NW], w1[NW];  // the two weight register sets
  // stage p's loads into ring slot S: x, weights, scales (LB = 4 + NW + 1 loads)
  auto batch = [&](int p, auto slot) {
    constexpr int S = decltype(slot)::value;
    uint8_t* const xd = S ? xl1 : xl0;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (void __attribute__((address_space(3)))*)(xd + 4 * (wave + 4 * j) * XROW), 16,
          xvo[j], p * XROW, 0, 0);
    u32x4* const wd = S ? w1 : w0;
    wd[0] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo0, p * 1024, 0);
    wd[1] = __builtin_amdgcn_raw_buffer_load_b128(wrs, wvo1, p * 1024, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        srs, (void __attribute__((address_space(3)))*)((S ? sl1 : sl0) + wave * 256), 4, svo,
        p * 64, 0, 0);
  };
  // correction operands b and -128 s of this wave's fragments (groups past G: zero)
  u32x4 Ab[NW][GJ], As[NW][GJ];
  auto corr = [&]() {
#pragma unroll
    for (int i = 0; i < NW; ++i)
#pragma unroll
      for (int jb = 0; jb < GJ; ++jb) {
        const bool gin = 32 * jb + 8 * c4 < G;
        const int64_t o = (int64_t)((f0 + i) * 16 + r16) * G + (gin ? 32 * jb + 8 * c4 : 0);
        Ab[i][jb] = *reinterpret_cast<const u32x4*>(bias + o);
        As[i][jb] = *reinterpret_cast<const u32x4*>(nsc + o);
        if (!gin) Ab[i][jb] = As[i][jb] = (u32x4){0u, 0u, 0u, 0u};
      }
  };

  if constexpr (XS) {  // the caller's split sums, 3 x 64 rows x G bf16, in 1 KiB copies
    const __amdgpu_buffer_rsrc_t grs = __builtin_amdgcn_make_buffer_rsrc(
        (void*)xsg, (short)0, 3 * MT * G * 2, 0x00020000);
    for (int c = wave; c < (3 * MT * G * 2 + 1023) / 1024; c += 4)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          grs, (void __attribute__((address_space(3)))*)(sxb + 1024 * c), 16, 1024 * c + 16 * lane,
          0, 0, 0);
  }
  batch(0, std::integral_constant<int, 0>{});
  wait_vm<0>();
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup", "global");

  f32x4 T[NW][MW];
#pragma unroll
  for (int i = 0; i < NW; ++i)
#pragma unroll
    for (int u = 0; u < MW; ++u) T[i][u] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  uint32_t nib = 0x000F000Fu;
  asm volatile("" : "+v"(nib));  // keep the nibble mask in a VGPR
  float pk[KT];
#pragma unroll
  for (int k = 0; k < KT; ++k) pk[k] = 0.f;

  // Stage p from ring slot S. kind 1: first issue stage p+1's loads into the
  // other slot; kind 2: issue the correction loads. last: no wait and barrier.
  auto stage = [&](int p, auto slot, auto kindc, auto lastc) {
    constexpr int S = decltype(slot)::value, kind = decltype(kindc)::value;
    constexpr bool last = decltype(lastc)::value;
    if constexpr (kind == 1) batch(p + 1, std::integral_constant<int, 1 - S>{});
    if constexpr (kind == 2) corr();
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* const cur = S ? xl1 : xl0;
    const u32x4* const wc = S ? w1 : w0;
#pragma unroll
    for (int gl = 0; gl < 2; ++gl) {
      u32x4 X[MW][2];
#pragma unroll
      for (int u = 0; u < MW; ++u)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = u * 16 + r16;
          const int ch = 8 * gl + 4 * h + c4;
          X[u][h] = *reinterpret_cast<const u32x4*>(&cur[row * XROW + ((ch ^ r16) << 4)]);
        }
      if constexpr (!XS) {
        // X_g of group 2p + gl, rows 16 wave + r16: lane group c4 keeps it when
        // (2 S + gl) == c4, in the newest shift-register slot
#pragma unroll
        for (int u = 0; u < MW; ++u)
          if (u == wave) {
            f32x4 a = mfma(ones, X[u][0], zero);
            a = mfma(ones, X[u][1], a);
            pk[KT - 1] = c4 == 2 * S + gl ? a[0] : pk[KT - 1];
          }
      }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        const u32x4 A0 = unpack_w(wc[i][2 * gl], nib), A1 = unpack_w(wc[i][2 * gl + 1], nib);
        const u32x4 sv = *reinterpret_cast<const u32x4*>((S ? sl1 : sl0) + wave * 256 + i * 64 + c4 * 16);
        float s[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) s[r] = gl ? bf_hi(sv[r]) : bf_lo(sv[r]);
#pragma unroll
        for (int u = 0; u < MW; ++u) {
          f32x4 a = mfma(A0, X[u][0], zero);
          a = mfma(A1, X[u][1], a);
#pragma unroll
          for (int r = 0; r < 4; ++r) T[i][u][r] = fmaf(s[r], a[r], T[i][u][r]);
        }
      }
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!last) {
      wait_vm<0>();  // this wave's copies of stage p + 1 (and its weights) have landed
      wait_lgkm0();
      __builtin_amdgcn_s_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "workgroup", "global");
    }
  };
  // a ring turn is two stages; the shift register moves down one slot per turn
  auto shift = [&]() {
#pragma unroll
    for (int k = 0; k + 1 < KT; ++k) pk[k] = pk[k + 1];
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using K2 = std::integral_constant<int, 2>;
  using NL = std::false_type;
  int p = 0;
#pragma nounroll
  for (; p < P - 2; p += 2) {
    if constexpr (!XS) shift();
    stage(p, S0{}, S1{}, NL{});
    stage(p + 1, S1{}, S1{}, NL{});
  }
  if constexpr (!XS) shift();
  stage(p, S0{}, S1{}, NL{});
  stage(p + 1, S1{}, K2{}, std::true_type{});
  wait_vm<0>();
  wait_lgkm0();
  if constexpr (!XS) {
    // turn t (of P / 2) sits in pk[KT - P/2 + t]: group 4t + c4 of rows 16 wave + r16
    float* const sx = reinterpret_cast<float*>(sxb);
    const int k0 = KT - P / 2;
#pragma unroll
    for (int k = 0; k < KT; ++k)
      if (k >= k0) sx[(4 * (k - k0) + c4) * MT + wave * 16 + r16] = pk[k];
  }
  lds_barrier();

  // sum_g (b_g - 128 s_g) X_g, X_g = hi + mid + lo exactly
#pragma unroll
  for (int u = 0; u < MW; ++u) {
    const int row = u * 16 + r16;
#pragma unroll
    for (int jb = 0; jb < GJ; ++jb) {
      const bool gin = 32 * jb + 8 * c4 < G;
      u32x4 hi, mid, lo;
      if constexpr (XS) {
        const uint16_t* const xsl = reinterpret_cast<const uint16_t*>(sxb);
        const int o = row * G + (gin ? 32 * jb + 8 * c4 : 0);
        hi = *reinterpret_cast<const u32x4*>(xsl + o);
        mid = *reinterpret_cast<const u32x4*>(xsl + MT * G + o);
        lo = *reinterpret_cast<const u32x4*>(xsl + 2 * MT * G + o);
        if (!gin) hi = mid = lo = (u32x4){0u, 0u, 0u, 0u};
      } else {
        const float* const sx = reinterpret_cast<const float*>(sxb);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          float v0 = 0.f, v1 = 0.f;
          if (gin) {
            v0 = sx[(32 * jb + 8 * c4 + e) * MT + row];
            v1 = sx[(32 * jb + 8 * c4 + e + 1) * MT + row];
          }
          const uint32_t h = f2bf2(v0, v1);
          const float r0 = v0 - bf_lo(h), r1 = v1 - bf_hi(h);
          const uint32_t md = f2bf2(r0, r1);
          hi[e >> 1] = h;
          mid[e >> 1] = md;
          lo[e >> 1] = f2bf2(r0 - bf_lo(md), r1 - bf_hi(md));
        }
      }
#pragma unroll
      for (int i = 0; i < NW; ++i) {
        f32x4 t = T[i][u];
        t = mfma(Ab[i][jb], hi, t);
        t = mfma(Ab[i][jb], mid, t);
        t = mfma(Ab[i][jb], lo, t);
        t = mfma(As[i][jb], hi, t);
        t = mfma(As[i][jb], mid, t);
        t = mfma(As[i][jb], lo, t);
        T[i][u] = t;
      }
    }
  }

#pragma unroll
  for (int u = 0; u < MW; ++u) {
    const int m = u * 16 + r16;
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

// Decode shapes (M <= 64). A work-group owns 64 columns (four 16-wide
// fragments) and the K slice of NW * SPW stages starting at stage
// NW * SPW * blockIdx.y; wave w takes SPW stages of it and computes partial
// sums of all 64 x 64 outputs of its stages. The NW partial tiles are added
// through LDS at the end in wave order, each wave finishing 16 / NW of the
// sixteen 16 x 16 tiles (correction and store).
//
// Roles: x is the MFMA A operand and the weights the B operand, so a lane
// holds D[m][n] for four rows m = 16u + 4c + i and one column n = r16 of the
// fragment, and the per-group scale it applies is a single number.
//
// x goes through LDS: every work-group reads all of x, and a load of 16 rows x
// 64 B (the MFMA operand layout) ran at less than half the rate of whole
// 128-B rows through a CU's vector memory path, so each wave copies its own
// x slice, one group (64 rows x 64 k) at a time, with loads of 8 rows x 128 B
// straight into LDS (no VGPRs), the 16-B chunks of a row XOR-swizzled by
// (row / 2) % 8 so that the operand reads (ds_read_b128 of 16 rows) are
// conflict-free. Two buffers per wave: group q + 2 is loaded while q + 1 is
// in flight and q is used. Only the wave itself reads its buffers, so the
// hand-off is a vmcnt wait, no barrier; the buffers are two separate arrays
// so the compiler can tell loads into one from reads of the other.
//
// X_g (the group sums of x) comes from MFMAs of x against 0/1 row selectors
// (the A operand, ones in rows 4u..4u+3 for the 16-row block u), chained so
// the four blocks land in different output rows and lane (r16, c) ends with
// X_g[16c + r16] in one register, stored to LDS after the loop (an LDS store
// in the loop would make the compiler wait for every LDS copy in flight).
//
// With one slice (gridDim.y == 1) the kernel writes bf16 y; with several it
// writes its f32 partial sums, correction of its own groups included, to
// part[blockIdx.y][m][n] (row stride Npad), and qlinear_sum_kernel (or the
// consumer of a deferred call) adds the slices in order and rounds once.
//
// With XS the group sums come split from the caller (xsg [3][64][K/64], hi,
// mid, lo: launch_add_norm's), one K slice only: no X_g products, no split.
template <int NW, int SPW, bool XS>
__global__ __launch_bounds__(64 * NW) void qlinear_decode_kernel(
    const uint16_t* __restrict__ x, int64_t xs, int M, int K, const u32x4* __restrict__ wp,
    const uint16_t* __restrict__ sp, const uint16_t* __restrict__ bias,
    const uint16_t* __restrict__ nsc, int N, uint16_t* __restrict__ y, int64_t ys,
    float* __restrict__ part, int Npad, const uint16_t* __restrict__ xsg) {
  constexpr int G = 2 * NW * SPW;  // groups of the slice
  constexpr int NG = 2 * SPW;      // groups of a wave
  constexpr int GJ = (G + 31) / 32;
  constexpr int TPW = 16 / NW;     // tiles each wave finishes
  constexpr int XR = 32 * GJ + 8;  // bf16 per row of the split X_g arrays (16 B pad)
  static_assert(NW == 4 || NW == 8, "16 tiles over the waves");
  // Per wave two x buffers of one group each (64 rows x 128 B, chunk-swizzled);
  // after the loop the wave's partial tiles (tiles 0-7 in xb0, 8-15 in xb1).
  __shared__ __align__(16) uint8_t xb0[NW][8192];
  __shared__ __align__(16) uint8_t xb1[NW][8192];
  __shared__ __align__(16) float sx[G * 64];          // X_g[m] at sx[g * 64 + m]
  __shared__ __align__(16) uint16_t xsp[3][64 * XR];  // X_g = hi + mid + lo, [m][g] bf16

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r16 = lane & 15, c4 = lane >> 4;
  const int P = K >> 7, Gtot = K >> 6;
  const int pslice = blockIdx.y * (NW * SPW);
  const int p0 = pslice + w * SPW;  // first stage of the wave
  const int fb = blockIdx.x * 4;    // first fragment of the work-group

  const u32x4* wsrc = wp + ((int64_t)fb * P + p0) * 64 + lane;
  // scales of column r16 of each fragment, groups 2p and 2p+1 (one dword)
  const uint32_t* ssrc = reinterpret_cast<const uint32_t*>(sp) + ((int64_t)fb * P + p0) * 16 + r16;
  // x rows M..63 read as zeros: the buffer ends with row M-1
  const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
      (void*)x, (short)0, (int)(((int64_t)(M - 1) * xs + K) * 2), 0x00020000);
  // group q of the wave into buffer bq: load i covers rows 8i..8i+7, lane L
  // row 8i + L/8 and chunk (L % 8) ^ ((row / 2) % 8), stored at byte 16 L
  const int drow = lane >> 3;
  auto copy_x = [&](int q, int bq) {
    uint8_t* const sb = bq ? xb1[w] : xb0[w];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int r = 8 * i + drow;
      const int c = (lane & 7) ^ ((4 * i + (drow >> 1)) & 7);
      const int voff = (int)((r * xs + 128 * p0 + 64 * q + 8 * c) * 2);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xrs, (void __attribute__((address_space(3)))*)(sb + i * 1024), 16, voff, 0, 0, 0);
    }
  };
  // chunk c (8 k) of row r in buffer bq
  auto x_chunk = [&](int bq, int r, int c) -> u32x4 {
    const uint8_t* const sb = bq ? xb1[w] : xb0[w];
    return *reinterpret_cast<const u32x4*>(sb + 128 * r + 16 * (c ^ ((r >> 1) & 7)));
  };

  // Issue order (the vmcnt waits below count it): x of groups 0 and 1, then
  // every weight and scale of the wave, then the correction operands.
  u32x4 wr[SPW][4];
  uint32_t sr[SPW][4];
  copy_x(0, 0);
  if (NG > 1) copy_x(1, 1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int s = 0; s < SPW; ++s)
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      // weights and scales are read once: nontemporal
      wr[s][f] = __builtin_nontemporal_load(wsrc + (int64_t)f * P * 64 + s * 64);
      sr[s][f] = __builtin_nontemporal_load(ssrc + (int64_t)f * P * 16 + s * 16);
    }
  // correction operands of the fragment this wave finishes (groups beyond the slice: zero)
  const int fo = (w * TPW) >> 2;
  u32x4 Ab[GJ], As[GJ];
#pragma unroll
  for (int j = 0; j < GJ; ++j) {
    const bool gin = 32 * j + 8 * c4 < G;
    const int64_t o = ((int64_t)(fb + fo) * 16 + r16) * Gtot + 2 * pslice + (gin ? 32 * j + 8 * c4 : 0);
    Ab[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(bias + o));
    As[j] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(nsc + o));
    if (!gin) Ab[j] = As[j] = (u32x4){0u, 0u, 0u, 0u};
  }
  // the caller's split group sums of the rows of the tiles this wave finishes
  u32x4 Xs[XS ? TPW : 1][3][GJ];
  if constexpr (XS) {
#pragma unroll
    for (int i = 0; i < TPW; ++i) {
      const int u = (w * TPW + i) & 3;
#pragma unroll
      for (int j = 0; j < GJ; ++j) {
        const bool gin = 32 * j + 8 * c4 < G;
        const int64_t o = (int64_t)(16 * u + r16) * Gtot + 2 * pslice + (gin ? 32 * j + 8 * c4 : 0);
#pragma unroll
        for (int k = 0; k < 3; ++k) {
          Xs[i][k][j] = *reinterpret_cast<const u32x4*>(xsg + (int64_t)k * 64 * Gtot + o);
          if (!gin) Xs[i][k][j] = (u32x4){0u, 0u, 0u, 0u};
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  // T[f][u]: D[m][n] for m = 16u + 4c4 + i, n = 16(fb+f) + r16
  f32x4 T[4][4];
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int u = 0; u < 4; ++u) T[f][u] = (f32x4){0.f, 0.f, 0.f, 0.f};
  const u32x4 ones = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};
  const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
  uint32_t nib = 0x000F000Fu;
  asm volatile("" : "+v"(nib));
  // sel1[u]: the A operand with ones in rows 4u..4u+3 (lane r16 supplies row r16)
  u32x4 sel1[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) sel1[u] = (r16 >> 2) == u ? ones : (u32x4){0u, 0u, 0u, 0u};
  float xgv[NG];
  constexpr int WS = 8 * SPW + 2 * GJ + (XS ? 3 * TPW * GJ : 0);  // weight, scale, correction loads

#pragma unroll
  for (int q = 0; q < NG; ++q) {
    const int b = q & 1, s = q >> 1, gl = q & 1;
    // x of group q in LDS: the vector-memory ops issued after its copy may be pending
    if (q == 0) wait_vm<(NG > 1 ? 8 : 0) + WS>();
    else if (q == 1) wait_vm<WS + (NG > 2 ? 8 : 0)>();
    else if (q + 1 < NG) wait_vm<8>();
    else wait_vm<0>();
    u32x4 X[2][4];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int u = 0; u < 4; ++u) X[j][u] = x_chunk(b, 16 * u + r16, 4 * j + c4);
    if constexpr (!XS) {  // D[n][m] += X_g[16u + m] for n in 4u..4u+3: lane (r16, c4) gets X_g[16 c4 + r16]
      f32x4 xg = zero;
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        xg = mfma(sel1[u], X[0][u], xg);
        xg = mfma(sel1[u], X[1][u], xg);
      }
      xgv[q] = xg[0];
    }
#pragma unroll
    for (int f = 0; f < 4; ++f) {
      const u32x4 A0 = unpack_w(wr[s][f][2 * gl], nib), A1 = unpack_w(wr[s][f][2 * gl + 1], nib);
      const float sc = gl ? bf_hi(sr[s][f]) : bf_lo(sr[s][f]);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        f32x4 a = mfma(X[0][u], A0, zero);
        a = mfma(X[1][u], A1, a);
#pragma unroll
        for (int i = 0; i < 4; ++i) T[f][u][i] = fmaf(sc, a[i], T[f][u][i]);
      }
    }
    if (q + 2 < NG) {  // buffer b is free once its reads have returned
      wait_lgkm0();
      copy_x(q + 2, b);
    }
    __builtin_amdgcn_sched_barrier(0);
  }

  if constexpr (!XS) {
#pragma unroll
    for (int q = 0; q < NG; ++q) sx[(2 * w * SPW + q) * 64 + 16 * c4 + r16] = xgv[q];
  }
  // partial tiles into the wave's own buffers (all its copies have landed and been read)
#pragma unroll
  for (int f = 0; f < 4; ++f)
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = 4 * f + u;
      reinterpret_cast<f32x4*>(t < 8 ? xb0[w] : xb1[w])[(t & 7) * 64 + lane] = T[f][u];
    }
  lds_barrier();

  // X_g split once per work-group: thread -> row m, four groups
  for (int idx = tid; !XS && idx < 64 * 8 * GJ; idx += 64 * NW) {
    const int m = idx & 63, g0 = 4 * (idx >> 6);
    uint32_t h2[2], m2[2], l2[2];
#pragma unroll
    for (int e = 0; e < 4; e += 2) {
      const float v0 = g0 + e < G ? sx[(g0 + e) * 64 + m] : 0.f;
      const float v1 = g0 + e + 1 < G ? sx[(g0 + e + 1) * 64 + m] : 0.f;
      const uint32_t h = f2bf2(v0, v1);
      const float q0 = v0 - bf_lo(h), q1 = v1 - bf_hi(h);
      const uint32_t md = f2bf2(q0, q1);
      h2[e >> 1] = h;
      m2[e >> 1] = md;
      l2[e >> 1] = f2bf2(q0 - bf_lo(md), q1 - bf_hi(md));
    }
    *reinterpret_cast<u32x2*>(&xsp[0][m * XR + g0]) = (u32x2){h2[0], h2[1]};
    *reinterpret_cast<u32x2*>(&xsp[1][m * XR + g0]) = (u32x2){m2[0], m2[1]};
    *reinterpret_cast<u32x2*>(&xsp[2][m * XR + g0]) = (u32x2){l2[0], l2[1]};
  }
  if constexpr (!XS) lds_barrier();

  const int n = (fb + fo) * 16 + r16;
#pragma unroll
  for (int i = 0; i < TPW; ++i) {
    const int t = w * TPW + i, u = t & 3;
    f32x4 acc = reinterpret_cast<const f32x4*>(t < 8 ? xb0[0] : xb1[0])[(t & 7) * 64 + lane];
#pragma unroll
    for (int v = 1; v < NW; ++v)
      acc += reinterpret_cast<const f32x4*>(t < 8 ? xb0[v] : xb1[v])[(t & 7) * 64 + lane];
    // sum_g (b_g - 128 s_g) X_g, X_g of rows 16u + r16 as the A operand
#pragma unroll
    for (int jb = 0; jb < GJ; ++jb) {
      const int o = (16 * u + r16) * XR + 32 * jb + 8 * c4;
      const u32x4 hi = XS ? Xs[XS ? i : 0][0][jb] : *reinterpret_cast<const u32x4*>(&xsp[0][o]);
      const u32x4 mid = XS ? Xs[XS ? i : 0][1][jb] : *reinterpret_cast<const u32x4*>(&xsp[1][o]);
      const u32x4 lo = XS ? Xs[XS ? i : 0][2][jb] : *reinterpret_cast<const u32x4*>(&xsp[2][o]);
      acc = mfma(hi, Ab[jb], acc);
      acc = mfma(mid, Ab[jb], acc);
      acc = mfma(lo, Ab[jb], acc);
      acc = mfma(hi, As[jb], acc);
      acc = mfma(mid, As[jb], acc);
      acc = mfma(lo, As[jb], acc);
    }
    const int m0 = 16 * u + 4 * c4;
    if (part != nullptr) {
      float* pr = part + ((int64_t)blockIdx.y * 64 + m0) * Npad + n;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (m0 + e < M) pr[(int64_t)e * Npad] = acc[e];
    } else if (n < N) {
      uint16_t* yr = y + (int64_t)m0 * ys + n;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        if (m0 + e < M) yr[(int64_t)e * ys] = f2bf(acc[e]);
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

template <int KT, bool XS>
hipError_t launch_head(const QLinearArgs& a) {
  hipLaunchKernelGGL((qlinear_head_kernel<KT, XS>), dim3(a.Npad / 128), dim3(256), 0, a.stream, a.x,
                     a.xs, a.M, a.K, reinterpret_cast<const uint16_t*>(a.wp), a.sp, a.bias, a.nsc,
                     a.N, a.Npad, a.y, a.ys, a.xsplit);
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
  // (out_proj: 2048 columns), and every K above 2048, split K into slices of
  // 1024 (K a multiple of 1024) or 512; very wide layers take the tiled kernel
  if (K <= 512 || (K <= 2048 && Npad / 64 >= 128) || Npad >= kWideDecodeN) return 1;
  return K % 1024 == 0 ? K / 1024 : K / 512;
}

// Tile choice: up to 64 rows (batched decode) qlinear_decode_kernel, whole K
// (K = 512, 1024, 2048) or K slices (narrow layers, and every K above 2048 --
// those always get a workspace); otherwise 64 x 128 tiles (prefill). Of the
// tilings swept at 16384 x 2048 -> 12352 (four waves each, 16-wide fragments
// per wave m x n: 4x4, 2x4, 4x2, 2x2, 2x4 in one row of waves, 1x4, 2x2 in
// one column), 2 x 4 fragments per wave in a 2 x 2 wave grid was fastest:
// about 200 VGPRs and 48 KB of LDS give two waves per SIMD (1.42 ms; 4 x 4
// with one wave per SIMD took 1.98 ms). Deeper x prefetch (two stages in
// registers) pushed it to one wave per SIMD and 2.06 ms; an XCD-aware tile
// order (each XCD's L2 holding its own weight columns) changed nothing.
//
// Decode kernel shapes (64 x 12352 x 2048 and 64 x 2048 x 4096, 30 distinct
// layers): eight waves of two stages for K = 2048 (four waves of four stages,
// one wave per SIMD, were 20% slower), and for the narrow layer four slices
// of 1024 on eight waves (eight slices of 512 on four waves: 8% slower, and
// twice the partials).
//
// Very wide layers at decode sizes (lm_head, 248,320 columns) re-read all of
// x per 64 columns in the decode kernel, 4x the weight bytes through L2.
// There a 64 x 128 tile with every wave holding all 64 rows and two column
// fragments (one row of four waves) took 140 us at M = 64, K = 2048, against
// 196 us for the decode kernel, 159 us for the 2 x 2 wave grid and 157 us for
// four column fragments per wave (256 VGPRs, one wave per SIMD). The same tile
// with x copied by DMA at three waves per SIMD took 128-130 us timed alone
// (142.7 for the register-staged form in the same harness; 137 with DMA at two
// waves per SIMD; the register-staged form forced to three waves spills and
// takes 182). qlinear_head_kernel, the DMA tile with its group sums kept in
// registers through the K loop and its scales copied by DMA, takes 94-96 us
// timed alone on weights that stream from HBM (106-112 for the DMA tile that
// stored the sums to LDS in the loop, on the same boxes), 90 us in the
// executor's step with the norm's split sums. Loads three stages ahead at two
// waves per SIMD (108-111 us) and eight-wave groups (104-105 us) were slower.
hipError_t launch_qlinear(const QLinearArgs& a) {
  if (a.defer) *a.defer = QPartial{};
  if (a.M <= 64 && a.Npad >= kWideDecodeN) {
    // buffer offsets of the packed weights are 32-bit; K is a multiple of 512
    if (a.K % 512 != 0 || a.K > 4096 || (int64_t)a.Npad * a.K / 2 > INT32_MAX)
      return launch_cfg<4, 2, 1, 4>(a);
    const bool xs = a.xsplit != nullptr;
    if (a.K <= 2048) return xs ? launch_head<8, true>(a) : launch_head<8, false>(a);
    return xs ? launch_head<16, true>(a) : launch_head<16, false>(a);
  }
  if (a.M <= 64) {
    const int ns = a.part ? qlinear_decode_slices(a.K, a.Npad) : 1;
    const int ksl = a.K / ns;  // K of a slice
    if (ksl == 512 || ksl == 1024 || ksl == 2048) {
      const u32x4* wp = reinterpret_cast<const u32x4*>(a.wp);
      const bool xs = a.xsplit != nullptr && ns == 1 && ksl == 2048;
      auto kern = xs            ? qlinear_decode_kernel<8, 2, true>
                  : ksl == 2048 ? qlinear_decode_kernel<8, 2, false>
                  : ksl == 1024 ? qlinear_decode_kernel<8, 1, false>
                                : qlinear_decode_kernel<4, 1, false>;
      const int threads = ksl == 512 ? 256 : 512;
      hipLaunchKernelGGL(kern, dim3(a.Npad / 64, ns), dim3(threads), 0, a.stream, a.x, a.xs, a.M,
                         a.K, wp, a.sp, a.bias, a.nsc, a.N, a.y, a.ys, ns > 1 ? a.part : nullptr,
                         a.Npad, xs ? a.xsplit : nullptr);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess || ns == 1) return e;
      if (a.defer) {  // the consumer adds the slices
        *a.defer = QPartial{a.part, ns, a.Npad};
        return hipSuccess;
      }
      const int64_t n4 = (int64_t)a.M * (a.Npad / 4);
      hipLaunchKernelGGL(qlinear_sum_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                         a.stream, a.part, ns, a.M, a.N, a.Npad, a.y, a.ys);
      return hipGetLastError();
    }
  }
  return launch_cfg<2, 4, 2, 2>(a);
}

}  // namespace gdn
