// gdn_decode.hip -- gfx950 decode kernels of the gated delta rule.
//
// Work decomposition: one work-group per (sequence, key head hk). The group
// owns the R = Hv/Hk value heads hv = hk*R + r that share hk's q/k (the GQA
// map hk = hv / (Hv/Hk) of metal_gdn.rs:14), so the fused kernel computes the
// q/k conv channels once and is the only writer of every conv channel it
// reads: no two work-groups touch the same conv-state bytes of a slot.
//
// Each 128x128 f32 tile (one slot, one value head) is held in VGPRs by a
// "tile team" of 256 threads (4 waves), 64 floats per thread:
//   lt = thread index in the team, grp = lt >> 3 (0..31), sub = lt & 7;
//   rows  dv = grp + 32*i            (i = 0..3)
//   cols  dk = 4*(sub + 8*j) + e     (j = 0..3, e = 0..3)
// A load instruction of one wave reads 8 rows x 128 contiguous bytes, so every
// fetched cache line is fully used; the dk-reductions of a row stay inside 8
// aligned lanes and are done with three DPP adds (sum8).
//
// Arithmetic (metal_gdn.rs:37-62): s *= g; kv = s.k; d = (v - kv)*beta;
// s += k d; y = s.q. The readout is taken from the decayed state in the same
// pass as kv, using s_new.q = (g s).q + d (k.q): one reduction phase per token
// instead of two dependent ones.

#include "gdn_common.h"

namespace gdn {

struct TileRegs {
  v4f s[4][4];
};

__device__ __forceinline__ void tile_load(TileRegs& t, const float* __restrict__ tile, int grp,
                                          int sub) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      t.s[i][j] = __builtin_nontemporal_load(
          reinterpret_cast<const v4f*>(tile + (grp + 32 * i) * kDk + 4 * (sub + 8 * j)));
}

__device__ __forceinline__ void tile_store(const TileRegs& t, float* __restrict__ tile, int grp,
                                           int sub) {
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_nontemporal_store(
          t.s[i][j], reinterpret_cast<v4f*>(tile + (grp + 32 * i) * kDk + 4 * (sub + 8 * j)));
}

__device__ __forceinline__ float dot4(const v4f& a, const v4f& b) {
  return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// One token on the register tile. kl/ql: k and q of the token in LDS (Dk
// floats each); vrow[i]: v at row grp+32i; kq = k.q over all of Dk. yrow[i]
// gets the output of row grp+32i (identical in the 8 lanes of a row group).
// k/q are read from LDS per column block (j outer) so that only 8 of them are
// live at a time; the compiler barrier between the passes makes the second
// pass re-read k instead of keeping 16 registers alive across the reduction.
__device__ __forceinline__ void tile_step(TileRegs& t, const float* kl, const float* ql, int sub,
                                          const float vrow[4], float g, float beta, float kq,
                                          float yrow[4]) {
  float kd[4] = {0.f, 0.f, 0.f, 0.f}, qd[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const v4f kj = *reinterpret_cast<const v4f*>(kl + 4 * (sub + 8 * j));
    const v4f qj = *reinterpret_cast<const v4f*>(ql + 4 * (sub + 8 * j));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v4f sv = t.s[i][j] * g;
      kd[i] += dot4(sv, kj);
      qd[i] += dot4(sv, qj);
      t.s[i][j] = sv;
    }
  }
  float delta[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    kd[i] = sum8(kd[i]);
    qd[i] = sum8(qd[i]);
    delta[i] = (vrow[i] - kd[i]) * beta;
    yrow[i] = qd[i] + delta[i] * kq;
  }
  asm volatile("" ::: "memory");
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const v4f kj = *reinterpret_cast<const v4f*>(kl + 4 * (sub + 8 * j));
#pragma unroll
    for (int i = 0; i < 4; ++i) t.s[i][j] += kj * delta[i];
  }
}

// Baked rms-norm weights (qwen3_5.rs:551-552): bf16(1/128) and bf16(128^-0.5).
constexpr float kQNormW = 0.0078125f;
constexpr float kKNormW = 0.08837890625f;
constexpr float kNormEps = 1e-6f;

// -------------------------------------------------------------------------
// Fused S=1 decode: conv update + silu + split + q/k rms-norm + gates +
// recurrence. grid (Hk, B), block 256*R.
//
// Load order: the small conv/gate inputs first, then the 64 KiB state tile.
// Waiting for the conv inputs leaves the state loads in flight through the
// conv and norm phases, whose barriers order LDS only (lds_barrier). At most
// 128 VGPRs (4 waves per SIMD) lets two 512-thread groups share a CU, so one
// group's state stores overlap the other's loads.
template <int R>
__global__ __launch_bounds__(256 * R) __attribute__((amdgpu_waves_per_eu(4))) void
decode_fused_kernel(float* __restrict__ state, uint16_t* __restrict__ conv,
                    const int32_t* __restrict__ slot_ids, int num_slots, int Hk,
                    const uint16_t* __restrict__ mixed, const uint16_t* __restrict__ ab,
                    const float* __restrict__ A_log, const float* __restrict__ dt_bias,
                    const uint16_t* __restrict__ conv_w, uint16_t* __restrict__ y,
                    uint32_t* __restrict__ status) {
  constexpr int NT = 256 * R;
  constexpr int NCH = (2 + R) * kDk;  // q, k of hk + v of R value heads
  constexpr int CPT = (NCH + NT - 1) / NT;
  const int hk = blockIdx.x, b = blockIdx.y;
  const int Hv = Hk * R;
  const int D = 2 * Hk * kDk + Hv * kDv;
  const int tid = threadIdx.x;
  const int slot = slot_ids[b];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }

  __shared__ float xs[NCH];
  __shared__ __align__(16) float qn[kDk];
  __shared__ __align__(16) float kn[kDk];
  __shared__ float red[8];
  __shared__ float gate_g[R], gate_beta[R];
  __shared__ uint16_t win_next[kConvK - 1][NCH];  // shifted conv window, stored at the end

  // global conv channel of the group's local channel c (q | k | v blocks)
  auto chan = [&](int c) {
    return c < kDk ? hk * kDk + c
                   : (c < 2 * kDk ? Hk * kDk + hk * kDk + (c - kDk)
                                  : 2 * Hk * kDk + hk * R * kDv + (c - 2 * kDk));
  };

  // 1. conv window, weights and gate inputs of the channels this thread owns
  uint16_t* cs = conv + (size_t)slot * (kConvK - 1) * D;
  uint16_t cwin[CPT][kConvK];
  uint2 cwt[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = tid + u * NT;
    const int gc = chan(c < NCH ? c : 0);
    cwt[u] = *reinterpret_cast<const uint2*>(conv_w + (size_t)gc * kConvK);
    cwin[u][0] = cs[gc];
    cwin[u][1] = cs[D + gc];
    cwin[u][2] = cs[2 * D + gc];
    cwin[u][3] = mixed[(size_t)b * D + gc];
  }
  float braw = 0.f, araw = 0.f, alog = 0.f, dtb = 0.f;
  if (tid < R) {
    const int h = hk * R + tid;
    braw = bf2f(ab[(size_t)b * 2 * Hv + h]);
    araw = bf2f(ab[(size_t)b * 2 * Hv + Hv + h]);
    alog = A_log[h];
    dtb = dt_bias[h];
  }

  // 2. the state tile of value head hv (stays in flight until tile_step)
  const int r = tid >> 8;
  const int lt = tid & 255, grp = lt >> 3, sub = lt & 7;
  const int hv = hk * R + r;
  float* tile = state + ((size_t)slot * Hv + hv) * kTileElems;
  TileRegs t;
  tile_load(t, tile, grp, sub);

  // 3. conv (qwen3_5.rs:602-610): bf16 products, f32 sum, silu. The shifted
  // window goes to LDS and is stored at the end of the kernel: a store issued
  // here would sit behind the state loads in the in-order vmcnt counter and
  // force waits on them.
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = tid + u * NT;
    if (c < NCH) {
      float acc = rbf(bf2f(cwin[u][0]) * bf2f((uint16_t)(cwt[u].x & 0xffffu)));
      acc += rbf(bf2f(cwin[u][1]) * bf2f((uint16_t)(cwt[u].x >> 16)));
      acc += rbf(bf2f(cwin[u][2]) * bf2f((uint16_t)(cwt[u].y & 0xffffu)));
      acc += rbf(bf2f(cwin[u][3]) * bf2f((uint16_t)(cwt[u].y >> 16)));
      xs[c] = silu_bf16(rbf(acc));
#pragma unroll
      for (int k = 0; k < kConvK - 1; ++k) win_next[k][c] = cwin[u][k + 1];
    }
  }
  // gates (compiled_ops.rs:30-43) on ab = [b | a]
  if (tid < R) {
    gate_beta[tid] = rbf(sigmoid_f32(braw));
    const float sp = logf(expf(araw + dtb) + 1.0f);
    gate_g[tid] = expf(-(expf(alog) * sp));
  }
  lds_barrier();

  // 4. q/k rms-norm (qwen3_5.rs:638-639): waves 0-1 hold q, waves 2-3 hold k.
  const int wave = tid >> 6, lane = tid & 63;
  if (tid < 2 * kDk) {
    const float v = xs[tid];
    const float ss = wave_sum(v * v);
    if (lane == 0) red[wave] = ss;
  }
  lds_barrier();
  if (tid < kDk) {
    const float rq = 1.0f / sqrtf((red[0] + red[1]) / (float)kDk + kNormEps);
    const float rk = 1.0f / sqrtf((red[2] + red[3]) / (float)kDk + kNormEps);
    const float qv = rbf(kQNormW * rbf(xs[tid] * rq));
    const float kv = rbf(kKNormW * rbf(xs[kDk + tid] * rk));
    qn[tid] = qv;
    kn[tid] = kv;
    const float p = wave_sum(qv * kv);
    if (lane == 0) red[4 + wave] = p;
  }
  lds_barrier();
  const float kq = red[4] + red[5];

  // 5. recurrence on the tile
  float vrow[4], yrow[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) vrow[i] = xs[2 * kDk + r * kDv + grp + 32 * i];
  tile_step(t, kn, qn, sub, vrow, gate_g[r], gate_beta[r], kq, yrow);
  tile_store(t, tile, grp, sub);
  uint16_t* yo = y + ((size_t)b * Hv + hv) * kDv;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (sub == i) yo[grp + 32 * i] = f2bf(yrow[i]);
  // 6. rolling conv state: window [s0 s1 s2 x] -> [s1 s2 x] in place (this
  // group is the only one touching these channels of the slot)
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = tid + u * NT;
    if (c < NCH) {
      const int gc = chan(c);
#pragma unroll
      for (int k = 0; k < kConvK - 1; ++k) cs[(size_t)k * D + gc] = win_next[k][c];
    }
  }
}

// -------------------------------------------------------------------------
// Recurrence on prepared q/k/v/g/beta for T tokens per sequence (the
// gated_delta_kernel contract, metal_gdn.rs:10-67), state in pool slots.
// grid (Hk, B), block 256*R.
template <int R>
__global__ __launch_bounds__(256 * R) void recurrent_kernel(
    float* __restrict__ state, const int32_t* __restrict__ slot_ids, int num_slots, int Hk, int T,
    const uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
    const uint16_t* __restrict__ v, const float* __restrict__ g,
    const uint16_t* __restrict__ beta, uint16_t* __restrict__ y, uint32_t* __restrict__ status) {
  constexpr int NT = 256 * R;
  const int hk = blockIdx.x, b = blockIdx.y;
  const int Hv = Hk * R;
  const int tid = threadIdx.x;
  const int slot = slot_ids[b];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
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
  TileRegs t;
  tile_load(t, tile, grp, sub);

  for (int tt = 0; tt < T; ++tt) {
    const size_t tok = (size_t)b * T + tt;
    if (tid < kDk) {
      const float qv = bf2f(q[(tok * Hk + hk) * kDk + tid]);
      const float kv = bf2f(k[(tok * Hk + hk) * kDk + tid]);
      qs[tid] = qv;
      ks[tid] = kv;
      const float p = wave_sum(qv * kv);
      if (lane == 0) red[wave] = p;
    }
    for (int c = tid; c < R * kDv; c += NT) vs[c] = bf2f(v[(tok * Hv + hk * R) * kDv + c]);
    if (tid < R) {
      gg[tid] = g[tok * Hv + hk * R + tid];
      bb[tid] = bf2f(beta[tok * Hv + hk * R + tid]);
    }
    __syncthreads();
    const float kq = red[0] + red[1];
    float vrow[4], yrow[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) vrow[i] = vs[r * kDv + grp + 32 * i];
    tile_step(t, ks, qs, sub, vrow, gg[r], bb[r], kq, yrow);
    uint16_t* yo = y + (tok * Hv + hv) * kDv;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (sub == i) yo[grp + 32 * i] = f2bf(yrow[i]);
    __syncthreads();
  }
  tile_store(t, tile, grp, sub);
}

// ------------------------------------------------------------ launchers --

template <int R>
static hipError_t launch_decode_r(const DecodeArgs& a) {
  dim3 grid(a.Hk, a.B);
  hipLaunchKernelGGL(decode_fused_kernel<R>, grid, dim3(256 * R), 0, a.stream, a.state, a.conv,
                     a.slot_ids, a.num_slots, a.Hk, a.mixed, a.ab, a.A_log, a.dt_bias, a.conv_w,
                     a.y, a.status);
  return hipGetLastError();
}

hipError_t launch_decode(const DecodeArgs& a) {
  switch (a.R) {
    case 1: return launch_decode_r<1>(a);
    case 2: return launch_decode_r<2>(a);
    case 4: return launch_decode_r<4>(a);
    default: return hipErrorInvalidValue;
  }
}

template <int R>
static hipError_t launch_recurrent_r(const RecurrentArgs& a) {
  dim3 grid(a.Hk, a.B);
  hipLaunchKernelGGL(recurrent_kernel<R>, grid, dim3(256 * R), 0, a.stream, a.state, a.slot_ids,
                     a.num_slots, a.Hk, a.T, a.q, a.k, a.v, a.g, a.beta, a.y, a.status);
  return hipGetLastError();
}

hipError_t launch_recurrent(const RecurrentArgs& a) {
  switch (a.R) {
    case 1: return launch_recurrent_r<1>(a);
    case 2: return launch_recurrent_r<2>(a);
    case 4: return launch_recurrent_r<4>(a);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace gdn
