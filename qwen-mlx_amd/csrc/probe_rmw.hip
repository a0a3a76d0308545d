// probe_rmw.hip -- measurement-only kernels behind bench.py --rmw-probe and
// --copy-floor (built into lib/libgdn_probe.so, not part of libgdn's
// interface).
//
// Plain read-modify-write of the decode step's state bytes with no gated delta
// arithmetic: n slots of slot_bytes each, every byte read and written once per
// launch (x 0.999f), in one of several access shapes. They bound what a decode
// launch of the same bytes can reach for a given access pattern and slot
// placement.
//
//   shape 0: units of unit_bytes, unit u = block u, slot-major (the whole chip
//            sweeps the slots in slot order, unit by unit)
//   shape 1: the same units in a seeded random order (perm)
//   shape 2: the decode kernel's access: one 128 KiB item per group (slot s,
//            item i of 16), 512 threads, 8 waves x 8 steps of 2 KiB pieces; the
//            16 items of a slot interleaved at 2 KiB (piece p of item i at
//            piece index 16p + i), groups dealt to XCDs in runs of items, the
//            wave's load pairs gap x 64 clocks apart
//   shape 3: shape 2 with contiguous 128 KiB items (item i at i x 128 KiB)
//            and groups dealt item-first (XCD x runs items x and x + 8 of every
//            slot), loads back to back: the previous decode kernel's access
//
// Every unit index is checked against the unit count and every slot id
// against num_slots on the host before launch; the kernels index only
// [pool, pool + num_slots * slot_bytes).
//
// gdn_probe_copy: a plain streaming copy (16 bytes per lane, four loads in
// flight per lane, a grid-stride loop), with or without nontemporal hints: the
// device's copy rate for a byte count, the floor of a kernel that reads and
// writes those bytes once (the prefill's qkv kernel).

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float v4f __attribute__((ext_vector_type(4)));

template <int NV>
__global__ __launch_bounds__(256) void rmw_units(float* __restrict__ pool, const int* __restrict__ ids,
                                                 int64_t slot_floats, int units_per_slot,
                                                 const int* __restrict__ perm) {
  const int u = perm ? perm[blockIdx.x] : (int)blockIdx.x;
  const int s = u / units_per_slot, part = u - s * units_per_slot;
  v4f* base = reinterpret_cast<v4f*>(pool + (size_t)ids[s] * slot_floats) + (size_t)part * (256 * NV);
  v4f r[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) r[i] = __builtin_nontemporal_load(base + i * 256 + threadIdx.x);
#pragma unroll
  for (int i = 0; i < NV; ++i) __builtin_nontemporal_store(r[i] * 0.999f, base + i * 256 + threadIdx.x);
}

template <bool INTERLEAVED>
__global__ __launch_bounds__(512) void rmw_items(float* __restrict__ pool, const int* __restrict__ ids,
                                                 int64_t slot_floats, int gap) {
  const int n = gridDim.x, L = blockIdx.x;
  int item;
  if (INTERLEAVED) {
    const int x = L & 7;
    item = x * (n >> 3) + min(x, n & 7) + (L >> 3);
  } else {
    item = L;  // XCD L % 8 runs items L % 16 in {x, x + 8} of every slot
  }
  const int s = item >> 4, i = item & 15;
  float* slot = pool + (size_t)ids[s] * slot_floats;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, q = lane >> 4, l = lane & 15;
  auto row = [&](int j) -> float* {
    const int p = 8 * j + wave;  // piece of the item, 4 rows of 512 B
    return slot + (INTERLEAVED ? ((size_t)p * 16 + i) * 512 : (size_t)i * 32768 + (size_t)p * 512) + q * 128;
  };
  v4f r[8][2];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    r[j][0] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(row(j) + 4 * l));
    r[j][1] = __builtin_nontemporal_load(reinterpret_cast<const v4f*>(row(j) + 64 + 4 * l));
    if (INTERLEAVED && j < 7) {
      // s_sleep takes an immediate: a gap of 0 (back to back) or 4 x 64 clocks
      if (gap > 0) __builtin_amdgcn_s_sleep(4);
    }
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    __builtin_nontemporal_store(r[j][0] * 0.999f, reinterpret_cast<v4f*>(row(j) + 4 * l));
    __builtin_nontemporal_store(r[j][1] * 0.999f, reinterpret_cast<v4f*>(row(j) + 64 + 4 * l));
  }
}

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// b[i] = a[i], i < n (16-byte units); every index below n.
template <bool NT>
__global__ __launch_bounds__(256) void copy_units(const u32x4* __restrict__ a, u32x4* __restrict__ b,
                                                  size_t n) {
  const size_t st = (size_t)gridDim.x * 256;
  size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  for (; i + 3 * st < n; i += 4 * st) {
    u32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = NT ? __builtin_nontemporal_load(a + i + j * st) : a[i + j * st];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (NT) __builtin_nontemporal_store(v[j], b + i + j * st);
      else b[i + j * st] = v[j];
    }
  }
  for (; i < n; i += st) b[i] = a[i];
}

}  // namespace

// Copies `bytes` (a multiple of 16, both pointers 16-byte aligned) from src to
// dst with `grid` groups of 256 threads (1 .. 2^20); nontemporal != 0 uses
// nontemporal loads and stores. Returns 0, or a negative value for bad
// arguments.
extern "C" int gdn_probe_copy(const void* src, void* dst, int64_t bytes, int grid, int nontemporal,
                              void* stream) {
  if (!src || !dst || bytes <= 0 || bytes % 16 != 0) return -1;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) % 16 != 0) return -1;
  if (grid < 1 || grid > (1 << 20)) return -2;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const size_t n = (size_t)bytes / 16;
  const u32x4* a = static_cast<const u32x4*>(src);
  u32x4* b = static_cast<u32x4*>(dst);
  if (nontemporal)
    hipLaunchKernelGGL((copy_units<true>), dim3(grid), dim3(256), 0, s, a, b, n);
  else
    hipLaunchKernelGGL((copy_units<false>), dim3(grid), dim3(256), 0, s, a, b, n);
  return hipGetLastError() == hipSuccess ? 0 : -8;
}

// pool: num_slots slots of slot_bytes; ids: n slot ids (device); perm: for
// shape 1, a permutation of the n * slot_bytes / unit_bytes units (device);
// lds_bytes: dynamic LDS reserved per group (limits groups per CU). Shapes 2-3
// need slot_bytes == 2 MiB. Returns 0, or a negative value for bad arguments.
extern "C" int gdn_probe_rmw(float* pool, int num_slots, int64_t slot_bytes, const int32_t* ids,
                             const int32_t* host_ids, int n, int shape, int unit_bytes,
                             const int32_t* perm, int lds_bytes, int gap, void* stream) {
  if (!pool || !ids || !host_ids || n <= 0 || slot_bytes <= 0 || slot_bytes % 16384 != 0) return -1;
  for (int k = 0; k < n; ++k)
    if (host_ids[k] < 0 || host_ids[k] >= num_slots) return -2;
  if (lds_bytes < 0 || lds_bytes > 160 * 1024) return -3;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int64_t slot_floats = slot_bytes / 4;
  if (shape == 0 || shape == 1) {
    if (unit_bytes != 4096 && unit_bytes != 16384) return -4;
    if (slot_bytes % unit_bytes != 0) return -4;
    const int64_t ups = slot_bytes / unit_bytes, nunits = ups * n;
    if (nunits > INT32_MAX) return -4;
    if (shape == 1 && !perm) return -5;
    const int* pm = shape == 1 ? perm : nullptr;
    if (unit_bytes == 4096)
      hipLaunchKernelGGL((rmw_units<1>), dim3((unsigned)nunits), dim3(256), lds_bytes, s, pool, ids,
                         slot_floats, (int)ups, pm);
    else
      hipLaunchKernelGGL((rmw_units<4>), dim3((unsigned)nunits), dim3(256), lds_bytes, s, pool, ids,
                         slot_floats, (int)ups, pm);
  } else if (shape == 2 || shape == 3) {
    if (slot_bytes != 2 * 1024 * 1024) return -6;
    if (shape == 2)
      hipLaunchKernelGGL((rmw_items<true>), dim3(16 * n), dim3(512), lds_bytes, s, pool, ids,
                         slot_floats, gap);
    else
      hipLaunchKernelGGL((rmw_items<false>), dim3(16 * n), dim3(512), lds_bytes, s, pool, ids,
                         slot_floats, gap);
  } else {
    return -7;
  }
  return hipGetLastError() == hipSuccess ? 0 : -8;
}
