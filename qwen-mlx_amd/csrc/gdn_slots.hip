// gdn_slots.hip -- slot-pool data movement: zero, gather (read), scatter
// (write) and slot-list validation.
//
// These replace the per-sequence state handling of the reference executor:
// zero-init of a missing cache (qwen3_5.rs:598-601,644-648), the concat of
// stack_caches (mlx_executor.rs:42-55,92-115) and the row views of
// unstack_caches (mlx_executor.rs:118-130). On the decode path no data moves
// at all (kernels address slots directly); these kernels serve admission,
// export and tests. All copies are bit-exact 16-byte moves.
//
// grid (Hv, n, nlayers), block 256: work-group (x, i, l) moves value-head
// tile x of slot slot_ids[i] in layer layer0 + l (64 KiB: Dv rows of 512 B,
// placed in the slot by state_row_offset) plus a 1/Hv share of that slot's
// conv state. Caller buffers hold the tiles in the reference's [Hv, Dv, Dk]
// order.

#include "gdn_common.h"

namespace gdn {

constexpr int kSlotThreads = 256;

__global__ __launch_bounds__(kSlotThreads) void slots_kernel(SlotArgs a) {
  const int hv = blockIdx.x, i = blockIdx.y, layer = a.layer0 + blockIdx.z;
  const int tid = threadIdx.x;
  const int slot = a.slot_ids[i];
  if ((unsigned)slot >= (unsigned)a.num_slots) {
    if (tid == 0 && hv == 0) flag_status(a.status, GDN_FLAG_BAD_SLOT);
    return;
  }
  // the slot's state; row dv of value head hv at state_row_offset(hv, dv)
  float4* sslot = reinterpret_cast<float4*>(a.layers.state[layer] + (size_t)slot * a.Hv * kTileElems);
  const int Hk = a.Hv / a.R;
  // 16-byte unit e of the (hv) tile in the caller's [Dv, Dk] layout
  auto unit = [&](int e) -> float4& {
    return sslot[(state_row_offset(hv, e / (kDk / 4), Hk, a.R) >> 2) + e % (kDk / 4)];
  };
  // conv state of the slot as 16-byte chunks; conv_elems*2 is a multiple of 16.
  const int conv_u4 = a.conv_elems / 8;
  uint4* cs = reinterpret_cast<uint4*>(a.layers.conv[layer] + (size_t)slot * a.conv_elems);
  // caller buffers are [n, ...] in the pool's per-slot layout; for a
  // multi-layer move they are [nlayers, n, ...].
  const size_t row = (size_t)blockIdx.z * a.n + i;
  if (a.op == SlotOp::kZero) {
    const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int e = tid; e < kTileElems / 4; e += kSlotThreads) unit(e) = z;
    const uint4 zc = make_uint4(0u, 0u, 0u, 0u);
    for (int e = hv * kSlotThreads + tid; e < conv_u4; e += a.Hv * kSlotThreads) cs[e] = zc;
  } else if (a.op == SlotOp::kRead) {
    if (a.state_buf) {
      float4* dst = reinterpret_cast<float4*>(a.state_buf + (row * a.Hv + hv) * kTileElems);
      for (int e = tid; e < kTileElems / 4; e += kSlotThreads) dst[e] = unit(e);
    }
    if (a.conv_buf) {
      uint4* dst = reinterpret_cast<uint4*>(a.conv_buf + row * a.conv_elems);
      for (int e = hv * kSlotThreads + tid; e < conv_u4; e += a.Hv * kSlotThreads) dst[e] = cs[e];
    }
  } else {
    if (a.state_buf) {
      const float4* src =
          reinterpret_cast<const float4*>(a.state_buf + (row * a.Hv + hv) * kTileElems);
      for (int e = tid; e < kTileElems / 4; e += kSlotThreads) unit(e) = src[e];
    }
    if (a.conv_buf) {
      const uint4* src = reinterpret_cast<const uint4*>(a.conv_buf + row * a.conv_elems);
      for (int e = hv * kSlotThreads + tid; e < conv_u4; e += a.Hv * kSlotThreads) cs[e] = src[e];
    }
  }
}

hipError_t launch_slots(const SlotArgs& a) {
  if (a.n <= 0 || a.nlayers <= 0) return hipSuccess;
  dim3 grid(a.Hv, a.n, a.nlayers);
  hipLaunchKernelGGL(slots_kernel, grid, dim3(kSlotThreads), 0, a.stream, a);
  return hipGetLastError();
}

// Range and uniqueness check of a slot-id list, one work-group. Pools of up to
// kBitmapSlots slots mark each id in an LDS bitmap (a second mark of the same
// bit is a duplicate), O(n); larger pools compare pairs, O(n^2).
constexpr int kBitmapWords = 16384;  // 64 KiB of LDS
constexpr int kBitmapSlots = kBitmapWords * 32;

__global__ __launch_bounds__(256) void validate_kernel(const int32_t* __restrict__ ids, int n,
                                                       int num_slots, uint32_t* status) {
  __shared__ uint32_t seen[kBitmapWords];
  if (num_slots <= kBitmapSlots) {
    const int words = (num_slots + 31) >> 5;
    for (int i = threadIdx.x; i < words; i += blockDim.x) seen[i] = 0u;
    __syncthreads();
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
      const int s = ids[i];
      if ((unsigned)s >= (unsigned)num_slots) {
        flag_status(status, GDN_FLAG_BAD_SLOT);
        continue;
      }
      const uint32_t bit = 1u << (s & 31);
      if (atomicOr(&seen[s >> 5], bit) & bit) flag_status(status, GDN_FLAG_DUP_SLOT);
    }
    return;
  }
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int s = ids[i];
    if ((unsigned)s >= (unsigned)num_slots) flag_status(status, GDN_FLAG_BAD_SLOT);
    for (int j = 0; j < i; ++j)
      if (ids[j] == s) {
        flag_status(status, GDN_FLAG_DUP_SLOT);
        break;
      }
  }
}

hipError_t launch_validate(const int32_t* slot_ids, int n, int num_slots, uint32_t* status,
                           hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(validate_kernel, dim3(1), dim3(256), 0, stream, slot_ids, n, num_slots,
                     status);
  return hipGetLastError();
}

}  // namespace gdn
