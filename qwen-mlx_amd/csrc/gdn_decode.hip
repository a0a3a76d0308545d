// gdn_decode.hip -- gfx950 decode kernels of the gated delta rule.
//
// Work decomposition: one work-group per (sequence, key head hk). The group
// owns the R = Hv/Hk value heads hv = hk*R + r that share hk's q/k (the GQA
// map hk = hv / (Hv/Hk) of metal_gdn.rs:14), so the fused decode kernel
// computes the q/k conv channels once and is the only writer of every conv
// channel it reads: no two work-groups touch the same conv-state bytes of a
// slot.
//
// The recurrence kernel (prepared q/k/v, T tokens) holds each 128x128 f32
// tile in a "tile team" of 256 threads, 64 floats per thread:
//   lt = thread index in the team, grp = lt >> 3 (0..31), sub = lt & 7;
//   rows  dv = grp + 32*i            (i = 0..3)
//   cols  dk = 4*(sub + 8*j) + e     (j = 0..3, e = 0..3)
// and reduces over dk inside 8 aligned lanes (three DPP adds, sum8). The
// fused decode kernel uses a row layout with 16 lanes per row instead (see
// decode_kernel).
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

// slot: the slot's state (Hv * Dv * Dk floats); rows of value head hv are
// addressed through state_row_offset.
__device__ __forceinline__ void tile_load(TileRegs& t, const float* __restrict__ slot, int hv,
                                          int Hk, int R, int grp, int sub) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float* row = slot + state_row_offset(hv, grp + 32 * i, Hk, R);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      t.s[i][j] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(row + 4 * (sub + 8 * j)));
  }
}

__device__ __forceinline__ void tile_store(const TileRegs& t, float* __restrict__ slot, int hv,
                                           int Hk, int R, int grp, int sub) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float* row = slot + state_row_offset(hv, grp + 32 * i, Hk, R);
#pragma unroll
    for (int j = 0; j < 4; ++j)
      __builtin_nontemporal_store(t.s[i][j], reinterpret_cast<v4f*>(row + 4 * (sub + 8 * j)));
  }
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
  float* sslot = state + (size_t)slot * Hv * kTileElems;
  TileRegs t;
  tile_load(t, sslot, hv, Hk, R, grp, sub);

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
  tile_store(t, sslot, hv, Hk, R, grp, sub);
}

// -------------------------------------------------------------------------
// Fused S=1 decode (conv update + silu + split + q/k rms-norm + gates +
// recurrence, optionally the RMSNormGated epilogue), one launch. 1D grid of
// B * Hk groups of 256*R threads.
//
// Items: item i = b*Hk + hk is (sequence b, key head hk). Its group owns the q/k
// conv channels of hk and the v channels of its R value heads, so it is the
// only reader and writer of those conv-state bytes of the slot.
//
// XCDs: the dispatcher deals work-groups to the 8 XCDs round-robin (group L
// runs on XCD L % 8). xcd_item gives each XCD a contiguous run of items, so the
// Hk items of one sequence run side by side on one XCD. With the slot layout of
// state_row_offset (the Hk items of a slot interleaved at 2 KiB) and the piece
// order below, those groups sweep one dense window of the slot together.
// Measured on 30 layers x 1024-slot pools, B = 64, over 8 seeded random slot
// sets: 46.7 us per launch (max 46.8; contiguous, every 8th and every 16th
// slot 46.7-47.9), against 50.4 us (max 51.5; every 8th slot 55.4) for
// contiguous 64 KiB tiles with groups dealt hk-first across XCDs.
//
// Rows: the item's R*Dv rows are 32R pieces of 4 rows. In step j (0..7) wave w
// of the 4R waves takes piece 4R*j + w, which lies in value head
// r = 4R*j/32 (the same for every wave of the step). Lanes 16q..16q+15 own row q
// of the piece; lane l holds columns 4l..4l+3 and 64+4l..64+4l+3. The two load
// instructions of a wave's step read one contiguous 2 KiB piece, and every
// dk-reduction is a 16-lane DPP sum.
//
// Load order: the conv window, weights and gate inputs first, then all 16
// state loads. Waiting for the conv inputs then leaves the state loads in
// flight (vmcnt counts in issue order) through the conv, gate and norm phases,
// whose barriers order LDS only. Results used by only some lanes are computed
// by all of them (or written to LDS by all of them): a value consumed only
// inside a divergent branch drags its loads, and their wait, into the branch
// behind the state loads.
__device__ __forceinline__ float conv1(uint16_t c0, uint16_t c1, uint16_t c2, uint16_t x, uint2 w) {
  float acc = rbf(bf2f(c0) * bf_lo(w.x));
  acc += rbf(bf2f(c1) * bf_hi(w.x));
  acc += rbf(bf2f(c2) * bf_lo(w.y));
  acc += rbf(bf2f(x) * bf_hi(w.y));
  return silu_bf16(rbf(acc));
}

// Gap between a wave's state load pairs in the fused decode, in units of 64
// clocks (s_sleep).
constexpr int kDecodeLoadGap = 4;

// Item of work-group L among n: XCD x = L % 8 takes items
// [x*(n/8) + min(x, n%8), ...) in order, one per group it receives.
__device__ __forceinline__ int xcd_item(int L, int n) {
  const int x = L & 7;
  return x * (n >> 3) + min(x, n & 7) + (L >> 3);
}

template <int R, bool GATED>
__global__ __launch_bounds__(256 * R) void decode_kernel(
    float* __restrict__ state, uint16_t* __restrict__ conv, const int32_t* __restrict__ slot_ids,
    int num_slots, int Hk, const uint16_t* __restrict__ mixed, int64_t xstride,
    const uint16_t* __restrict__ ab, int64_t ab_stride, const float* __restrict__ A_log,
    const float* __restrict__ dt_bias, const uint16_t* __restrict__ conv_w,
    uint16_t* __restrict__ y, const uint16_t* __restrict__ norm_w, float norm_eps,
    uint16_t* __restrict__ out, uint32_t* __restrict__ status) {
  constexpr int NT = 256 * R, NW = 4 * R;
  constexpr int NCH = (2 + R) * kDk;
  constexpr int CPT = (NCH + NT - 1) / NT;
  const int item = xcd_item(blockIdx.x, gridDim.x);
  const int b = item / Hk, hk = item - b * Hk;
  const int Hv = Hk * R;
  const int D = 2 * Hk * kDk + Hv * kDv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l = lane & 15, q = lane >> 4;
  const int slot = slot_ids[b];
  if ((unsigned)slot >= (unsigned)num_slots) {
    if (tid == 0) flag_status(status, GDN_FLAG_BAD_SLOT);
    return;
  }
  __shared__ float xs[CPT * NT];
  __shared__ __align__(16) float qk[2][kDk];
  __shared__ float red[8];
  __shared__ float gsh[R][2];
  // RMSNormGated staging: silu(z) and w per (head, row), y of the rows, and the
  // per-wave sums of y^2 of each head
  __shared__ float zsil[GATED ? R * kDv : 1], wsh[GATED ? R * kDv : 1], ysh[GATED ? R * kDv : 1];
  __shared__ float ysq[R][NW];
  auto chan = [&](int c) {
    return c < kDk ? hk * kDk + c
                   : (c < 2 * kDk ? Hk * kDk + hk * kDk + (c - kDk)
                                  : 2 * Hk * kDk + hk * R * kDv + (c - 2 * kDk));
  };
  const uint16_t* xrow = mixed + (size_t)b * xstride;

  // 1. conv window, weights and gate inputs (and the gate's z and norm
  // weight of the thread's rows), then the state pieces
  uint16_t* cs = conv + (size_t)slot * (kConvK - 1) * D;
  uint2 cw[CPT];
  uint16_t c0[CPT], c1[CPT], c2[CPT], cx[CPT];
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = tid + u * NT;
    const int gc = chan(c < NCH ? c : 0);
    cw[u] = *reinterpret_cast<const uint2*>(conv_w + (size_t)gc * kConvK);
    c0[u] = cs[gc];
    c1[u] = cs[D + gc];
    c2[u] = cs[2 * D + gc];
    cx[u] = xrow[gc];
  }
  const int gr = tid & (R - 1), gh = hk * R + gr;
  const float alog = A_log[gh], dtb = dt_bias[gh];
  const uint16_t braw = ab[(size_t)b * ab_stride + gh], araw = ab[(size_t)b * ab_stride + Hv + gh];
  // gate inputs of (head hk*R + e/Dv, row e%Dv), e = t mod R*Dv: z follows
  // q|k|v in the merged row, so the R heads' z are contiguous
  uint16_t zr = 0, wr = 0;
  if constexpr (GATED) {
    const int e = tid & (R * kDv - 1);
    zr = xrow[D + hk * R * kDv + e];
    wr = norm_w[e & (kDv - 1)];
  }
  __builtin_amdgcn_sched_barrier(0);
  // step j: piece NW*j + wave = value head r_of(j), row dv_of(j) of that head
  auto r_of = [](int j) { return NW * j / 32; };
  auto dv_of = [&](int j) { return kPieceRows * ((NW * j + wave) & 31) + q; };
  float* sslot = state + (size_t)slot * Hv * kTileElems;
  float* rows[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) rows[j] = sslot + state_row_offset(hk * R + r_of(j), dv_of(j), Hk, R);
  // The wave's 8 load pairs go out kDecodeLoadGap x 64 clocks apart rather than
  // back to back: with every group of the chip issuing its 128 KiB in one
  // burst the launch measured 48.5 us; spaced, 46.7 us (gaps of 2-16 x 64
  // clocks all within 0.1 us; 32 x 64 clocks: 50.9 us).
  v4f s[8][2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    s[j][0] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(rows[j] + 4 * l));
    s[j][1] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(rows[j] + 64 + 4 * l));
    if (j < 7) __builtin_amdgcn_s_sleep(kDecodeLoadGap);
  }
  __builtin_amdgcn_sched_barrier(0);

  // 2. conv (qwen3_5.rs:602-610), gates (compiled_ops.rs:30-43) on ab = [b | a]
#pragma unroll
  for (int u = 0; u < CPT; ++u) xs[tid + u * NT] = conv1(c0[u], c1[u], c2[u], cx[u], cw[u]);
  {
    const float sp = logf(expf(bf2f(araw) + dtb) + 1.0f);
    gsh[gr][0] = expf(-(expf(alog) * sp));
    gsh[gr][1] = rbf(sigmoid_f32(bf2f(braw)));
  }
  if constexpr (GATED) {  // threads t and t + R*Dv write the same values
    zsil[tid & (R * kDv - 1)] = silu_bf16(bf2f(zr));
    wsh[tid & (R * kDv - 1)] = bf2f(wr);
  }
  lds_barrier();
  // 3. q/k rms-norm (qwen3_5.rs:638-639): waves 0-1 hold q, waves 2-3 hold k
  if (tid < 2 * kDk) {
    const float v = xs[tid];
    const float ss = wave_sum(v * v);
    if (lane == 0) red[wave] = ss;
  }
  lds_barrier();
  if (tid < 2 * kDk) {
    const float rn =
        1.0f / sqrtf((wave < 2 ? red[0] + red[1] : red[2] + red[3]) / (float)kDk + kNormEps);
    qk[tid >> 7][tid & (kDk - 1)] = rbf((tid < kDk ? kQNormW : kKNormW) * rbf(xs[tid] * rn));
  }
  lds_barrier();

  // 4. recurrence on the rows
  const v4f qa = *reinterpret_cast<const v4f*>(&qk[0][4 * l]);
  const v4f qb = *reinterpret_cast<const v4f*>(&qk[0][64 + 4 * l]);
  const v4f ka = *reinterpret_cast<const v4f*>(&qk[1][4 * l]);
  const v4f kb = *reinterpret_cast<const v4f*>(&qk[1][64 + 4 * l]);
  const float kq = sum16(dot4(ka, qa) + dot4(kb, qb));
  const size_t ybase = ((size_t)b * Hv + hk * R) * kDv;
  float yb[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = r_of(j), dv = dv_of(j);
    const float g = gsh[r][0], beta = gsh[r][1];
    const v4f a0 = s[j][0] * g, a1 = s[j][1] * g;
    const float kd = sum16(dot4(a0, ka) + dot4(a1, kb));
    const float qd = sum16(dot4(a0, qa) + dot4(a1, qb));
    const float d = (xs[2 * kDk + r * kDv + dv] - kd) * beta;
    __builtin_nontemporal_store(a0 + ka * d, reinterpret_cast<v4f*>(rows[j] + 4 * l));
    __builtin_nontemporal_store(a1 + kb * d, reinterpret_cast<v4f*>(rows[j] + 64 + 4 * l));
    yb[j] = rbf(qd + d * kq);
    if (y != nullptr && l == 0) y[ybase + r * kDv + dv] = f2bf(yb[j]);
  }

  // 5. RMSNormGated epilogue (qwen3_5.rs:660-665): out = silu(z) *
  // rms_norm(y, w, eps) over each head's Dv rows. Per wave and head, the sum
  // of y^2 over the wave's rows of that head (its steps, then the 4 lane
  // groups); y staged in LDS; after the barrier thread t < R*Dv writes row
  // t%Dv of head hk*R + t/Dv (coalesced), adding the NW wave sums in order.
  if constexpr (GATED) {
    float ss[R];
#pragma unroll
    for (int r = 0; r < R; ++r) ss[r] = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) ss[r_of(j)] += yb[j] * yb[j];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      ss[r] += __shfl_xor(ss[r], 16, 64);
      ss[r] += __shfl_xor(ss[r], 32, 64);
      if (lane == 0) ysq[r][wave] = ss[r];
    }
    if (l == 0) {
#pragma unroll
      for (int j = 0; j < 8; ++j) ysh[r_of(j) * kDv + dv_of(j)] = yb[j];
    }
    lds_barrier();
    if (tid < R * kDv) {
      const int h = tid / kDv;
      float tot = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) tot += ysq[h][w];
      const float rn = 1.0f / sqrtf(tot / (float)kDv + norm_eps);
      const float normed = rbf(wsh[tid] * rbf(ysh[tid] * rn));
      out[ybase + tid] = f2bf(zsil[tid] * normed);
    }
  }

  // 6. rolling conv state: window [s0 s1 s2 x] -> [s1 s2 x] in place (this
  // group's channels only)
#pragma unroll
  for (int u = 0; u < CPT; ++u) {
    const int c = tid + u * NT;
    if (c < NCH) {
      const int gc = chan(c);
      cs[gc] = c1[u];
      cs[D + gc] = c2[u];
      cs[2 * D + gc] = cx[u];
    }
  }
}

// ------------------------------------------------------------ launchers --

// Occupancy of the fused decode at R = 2: one 512-thread group per CU. The
// launch reserves 80 KB of LDS per group (unused; the CU has 160 KB), so a
// second group cannot start beside the first. Measured on 30 layers x B = 64
// over 8 random slot sets: 46.7 us per launch against 48.4 us with two groups
// per CU (the same results bit for bit).
constexpr size_t kDecodeOccupancyLds = 80 * 1024;

template <int R>
static hipError_t launch_decode_r(const DecodeArgs& a) {
  const size_t lds = R == 2 ? kDecodeOccupancyLds : 0;
  if (a.out)
    hipLaunchKernelGGL((decode_kernel<R, true>), dim3(a.Hk * a.B), dim3(256 * R), lds, a.stream,
                       a.state, a.conv, a.slot_ids, a.num_slots, a.Hk, a.mixed, a.xstride, a.ab, a.ab_stride,
                       a.A_log, a.dt_bias, a.conv_w, a.y, a.norm_w, a.norm_eps, a.out, a.status);
  else
    hipLaunchKernelGGL((decode_kernel<R, false>), dim3(a.Hk * a.B), dim3(256 * R), lds, a.stream,
                       a.state, a.conv, a.slot_ids, a.num_slots, a.Hk, a.mixed, a.xstride, a.ab, a.ab_stride,
                       a.A_log, a.dt_bias, a.conv_w, a.y, a.norm_w, a.norm_eps, a.out, a.status);
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
