// gdn_common.h -- shared definitions of libgdn's gfx950 kernels and host code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gdn.h"

namespace gdn {

// Compiled kernel family: Dk = Dv = 128, conv width 4. The value/key head
// ratio R = Hv / Hk is a template parameter (1, 2 or 4).
constexpr int kDk = 128;
constexpr int kDv = 128;
constexpr int kConvK = 4;
constexpr int kTileElems = kDv * kDk;  // one (slot, value head) recurrent tile

// Recurrent state layout inside one slot (Hv * Dv * Dk floats). The R = Hv/Hk
// value heads of key head hk form the item of hk: R * Dv rows, item row
// ir = r * Dv + dv for hv = hk * R + r. Item rows are cut into pieces of 4 rows
// (kPieceRows * Dk floats = 2 KiB), and piece p of key head hk is stored at
// piece index p * Hk + hk of the slot: the Hk items of a slot interleave at
// 2 KiB. Work-groups that stream the items of one slot side by side, in
// piece order, then sweep one dense window of the slot instead of Hk separate
// 128 KiB regions. A row (Dk floats) stays contiguous.
constexpr int kPieceRows = 4;
__host__ __device__ __forceinline__ size_t state_row_offset(int hv, int dv, int Hk, int R) {
  const int hk = hv / R, ir = (hv - hk * R) * kDv + dv;
  return ((size_t)(ir / kPieceRows) * Hk + hk) * (kPieceRows * kDk) + (size_t)(ir % kPieceRows) * kDk;
}

// Native 4 x f32 vector (16-byte loads/stores, usable with the nontemporal
// builtins).
typedef float v4f __attribute__((ext_vector_type(4)));

// Per-layer device pointers handed to kernels that span several layers.
struct LayerPtrs {
  float** state;      // [L] -> [num_slots, Hv, Dv, Dk]
  uint16_t** conv;    // [L] -> [num_slots, K-1, D]
};

// ------------------------------------------------------------------ bf16 --
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// Round to nearest even on v_cvt_pk_bf16_f32. For every non-NaN f32 bit
// pattern this equals the integer RNE (u + 0x7fff + ((u >> 16) & 1)) >> 16
// (checked exhaustively over all 2^32 patterns on gfx950); NaN stays NaN.
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint16_t f2bf(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }

// Two values in one conversion: a in the low half, b in the high half.
__device__ __forceinline__ uint32_t f2bf2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ float bf_lo(uint32_t v) { return __uint_as_float(v << 16); }
__device__ __forceinline__ float bf_hi(uint32_t v) { return __uint_as_float(v & 0xffff0000u); }

__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }
// rbf of two values with one conversion
__device__ __forceinline__ void rbf2(float& a, float& b) {
  const uint32_t p = f2bf2(a, b);
  a = bf_lo(p);
  b = bf_hi(p);
}

// MLX's f32 sigmoid: 1/(1+exp(-|x|)), mirrored for x < 0.
__device__ __forceinline__ float sigmoid_f32(float x) {
  float y = 1.0f / (1.0f + expf(-fabsf(x)));
  return x < 0.0f ? 1.0f - y : y;
}

// silu on a bf16 value with each elementwise op rounded to bf16.
__device__ __forceinline__ float silu_bf16(float x) { return rbf(x * rbf(sigmoid_f32(x))); }

// --------------------------------------------------------- lane reductions --
// DPP moves within a 16-lane row: quad_perm xor-1 / xor-2, and row_half_mirror
// (lane i <- lane 7-i inside each group of 8).
__device__ __forceinline__ float dpp_quad_xor1(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
}
__device__ __forceinline__ float dpp_half_mirror(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
}

// Sum over the 8 aligned lanes (lane & ~7) of a wave; every lane of the group
// receives the same bits.
__device__ __forceinline__ float sum8(float v) {
  v += dpp_quad_xor1(v);
  v += dpp_quad_xor2(v);
  v += dpp_half_mirror(v);
  return v;
}

// Sum over the 16 lanes of a DPP row (every lane receives the sum).
__device__ __forceinline__ float sum16(float v) {
  v = sum8(v);
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
}

// Sum over a full 64-lane wave (result in every lane).
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Work-group barrier that orders LDS only. Global loads issued before it stay
// in flight (a plain __syncthreads() would wait for every outstanding vector
// memory operation). Use it only where threads communicate through LDS.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// A pointer that is the same in every lane of the wave, moved to SGPRs so that
// loads can use scalar-base + 32-bit lane-offset addressing.
template <typename T>
__device__ __forceinline__ T* wave_uniform(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(v >> 32));
  return reinterpret_cast<T*>(((uint64_t)hi << 32) | lo);
}

__device__ __forceinline__ void flag_status(uint32_t* status, uint32_t bit) {
  if (status) atomicOr(status, bit);
}

}  // namespace gdn

// ------------------------------------------------- host launch interface --
namespace gdn {

struct DecodeArgs {
  int R, Hk, B, num_slots;
  float* state;
  uint16_t* conv;
  const int32_t* slot_ids;
  const uint16_t* mixed;   // [B, xstride] rows: q|k|v in the first D columns (then z if gated)
  int64_t xstride;         // row stride of mixed in elements (D, or the merged qkvz width)
  const uint16_t* ab;
  int64_t ab_stride;       // row stride of ab in elements (>= 2*Hv)
  const float* A_log;
  const float* dt_bias;
  const uint16_t* conv_w;
  uint16_t* y;             // recurrence output [B,Hv,Dv]; may be null when out is set
  const uint16_t* norm_w;  // RMSNormGated weight [Dv] (gated only)
  float norm_eps;
  uint16_t* out;           // gated output [B,Hv,Dv]; null = no epilogue
  uint32_t* status;
  hipStream_t stream;
};

struct RecurrentArgs {
  int R, Hk, B, T, num_slots;
  float* state;
  const int32_t* slot_ids;
  const uint16_t *q, *k, *v;
  const float* g;
  const uint16_t* beta;
  uint16_t* y;
  uint32_t* status;
  hipStream_t stream;
};

enum class SlotOp { kZero = 0, kRead = 1, kWrite = 2 };

struct SlotArgs {
  SlotOp op;
  LayerPtrs layers;     // device arrays of per-layer base pointers
  int layer0, nlayers;  // layers [layer0, layer0 + nlayers)
  int n, num_slots, Hv, R, conv_elems;  // R = Hv/Hk; conv_elems = (K-1)*D per slot
  const int32_t* slot_ids;
  float* state_buf;     // read: destination [n,...]; write: source
  uint16_t* conv_buf;
  uint32_t* status;
  hipStream_t stream;
};

struct PrefillArgs {
  int R, Hk, nseq, total_tokens, num_slots;
  float* state;
  uint16_t* conv;
  const int32_t* slot_ids;
  const int32_t* cu_seqlens;
  const uint16_t* mixed;  // [T, xstride]: q|k|v in columns [0, D), z (gated) in [D, D + Hv*Dv)
  int64_t xstride;
  const uint16_t* ab;     // [T, ab_stride]: b|a in the first 2*Hv columns
  int64_t ab_stride;
  const float* A_log;
  const float* dt_bias;
  const uint16_t* conv_w;
  uint16_t* y;            // [T, Hv, Dv]; may be null when out is set
  const uint16_t* norm_w; // RMSNormGated epilogue (out != null): weight [Dv], eps
  float norm_eps;
  uint16_t* out;          // [T, Hv, Dv] = silu(z) * rms_norm(y), or null
  uint32_t* status;
  int waves;             // prefill_chunk_waves of the call (8: fused chunk kernel)
  void* workspace;       // device scratch sized by prefill_workspace_bytes
  size_t workspace_bytes;
  hipStream_t stream;
  // Pipelined split path: `segments` (> 1) token segments over a second
  // stream of the caller's device with kPrefillPipeEvents events; aux null:
  // one pass.
  hipStream_t aux;
  hipEvent_t* events;
  int segments;
};
constexpr int kPrefillPipeSegmentsMax = 8;
constexpr int kPrefillPipeEvents = kPrefillPipeSegmentsMax + 2;

// 4-bit affine-quantized linear layer (gdn_qlinear.hip).
struct QLinearPackArgs {
  const uint32_t* w;  // MLX part: [N, K/8]
  const uint16_t* s;  // [N, K/64]
  const uint16_t* b;  // [N, K/64]
  int N, K, frag0;    // part rows, input width, first 16-row fragment in the merged matrix
  void* wp;           // packed weights of the merged matrix
  uint16_t* sp;       // packed scales
  uint16_t* bias;     // [Npad, K/64]
  uint16_t* nsc;      // [Npad, K/64] = -128 * scales
  hipStream_t stream;
};

// f32 K-slice partials that a decode-sized qlinear call left for its consumer
// to add: element (slice sl, row m, column n) at part[(sl * 64 + m) * Npad + n].
// The sum over sl = 0, 1, ..., nslice - 1 in that order, rounded once to bf16,
// is the call's output. nslice == 0: nothing pending (the call wrote y).
struct QPartial {
  const float* part = nullptr;
  int nslice = 0;
  int Npad = 0;
};

struct QLinearArgs {
  const uint16_t* x;  // [M, xs] bf16
  int64_t xs;
  int M, K, N, Npad;
  const void* wp;
  const uint16_t* sp;
  const uint16_t* bias;
  const uint16_t* nsc;
  uint16_t* y;        // [M, ys] bf16
  int64_t ys;
  float* part;        // K-slice partials [slices][64][Npad] f32 (decode shapes), or null
  QPartial* defer;    // non-null: a K-sliced call skips its slice sum and describes the
                      // partials here instead of writing y (nslice = 0 when y was written)
  const uint16_t* xsplit;  // or null: x's 64-column group sums as three bf16 parts
                           // [3][64][K/64] (launch_add_norm's), used by decode shapes
  hipStream_t stream;
};

hipError_t launch_qlinear_pack(const QLinearPackArgs& a);
hipError_t launch_qlinear(const QLinearArgs& a);
// K slices the decode path uses for a layer (1 = no partials workspace needed).
int qlinear_decode_slices(int K, int Npad);

hipError_t launch_decode(const DecodeArgs& a);
hipError_t launch_recurrent(const RecurrentArgs& a);
hipError_t launch_slots(const SlotArgs& a);
hipError_t launch_validate(const int32_t* slot_ids, int n, int num_slots, uint32_t* status,
                           hipStream_t stream);
int prefill_chunk_waves(int R, int Hk, int nseq, int total_tokens);
// Segments of a pipelined prefill call on the path `waves` picked, whose
// chunk kernel has `groups` work-groups, on a device of `cus` CUs (1: one
// pass, no second stream).
int prefill_pipeline_segments(int waves, int total_tokens, int groups, int cus);
size_t prefill_workspace_bytes(int R, int Hk, int total_tokens, int nseq, int waves, bool y_scratch);
size_t prefill_workspace_reserve_bytes(int R, int Hk, int max_tokens);
// Fixed per-device workspace of gdn_prefill_varlen_noalloc (gdn_prefill.hip).
size_t noalloc_scratch_bytes();
hipError_t noalloc_scratch(void** out);
hipError_t launch_prefill(const PrefillArgs& a);

// Attention step on the paged KV cache (gdn_attn.hip).
struct AttnArgs {
  int T, Hq, Hkv, P, max_pages, rot_dim;
  int NC, kpw;             // chunks of work in the step, chunks per worker
  bool stream_keys;        // each block read about once (non-temporal loads)
  float eps, log2_base;
  const uint16_t* q_full;  // [T, qs]: per query head 256 query then 256 gate values
  int64_t qs;
  const uint16_t* k;       // [T, ks]: Hkv x 256
  int64_t ks;
  const uint16_t* v;       // [T, vs]
  int64_t vs;
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  const int32_t* meta;     // [3][T]: slot, position, page of each token
  const int32_t* tokseg;   // [2][T]: token group, first column in the group
  const int32_t* grp;      // [groups][4]: first token, tokens, first position, slot
  const int32_t* seg;      // [groups * Hkv][4]: first chunk, chunks, -, -
  const int32_t* wseg;     // [P]: segment of each worker's first chunk
  int32_t* ptab;           // [num_slots][max_pages] page table
  uint16_t* pages;         // this layer's pages [num_pages][2][Hkv][16384]
  uint16_t* out;           // [T, os]: Hq x 256 gated attention rows
  int64_t os;
  void* workspace;         // attn_workspace_bytes(T, Hq, NC)
  hipStream_t stream;
};
size_t attn_workspace_bytes(int T, int Hq, int64_t chunks);
int attn_chunk_blocks();  // 16-key blocks per chunk
hipError_t launch_attn(const AttnArgs& a);
// A sequence's cached rows of one layer into [Hkv][len][256] K and V arrays.
hipError_t launch_kv_gather(const uint16_t* pages, const int32_t* prow, int Hkv, int64_t len,
                            uint16_t* k_out, uint16_t* v_out, hipStream_t s);

// Sets the calling thread's gdn_last_error() message and returns code.
gdn_status set_error(gdn_status code, const char* msg);

// Executor model-body kernels (gdn_exec.hip).
hipError_t launch_embed(const uint16_t* table, const int32_t* tok, int n, int vocab, int hidden,
                        uint16_t* h, hipStream_t s);
// gdn_qlinear_forward and gdn_layer_decode with the option to leave the
// projection's K-slice partials pending (defer non-null): a decode-sized
// projection that splits K then skips its slice sum, writes nothing to y and
// describes the partials in *defer for launch_add_norm to add; otherwise it
// writes y and sets defer->nslice = 0. The partials sit in the projection's
// own workspace until its next call.
gdn_status qlinear_forward(const gdn_qlinear* q, const uint16_t* x, int64_t x_stride, int32_t M,
                           uint16_t* y, int64_t y_stride, void* stream, QPartial* defer,
                           const uint16_t* xsplit = nullptr);
// Bumped each time the pool's layer-activation buffer is reallocated (a graph
// that captured gdn::layer_decode holds the old buffer's address).
uint64_t pool_act_generation(const gdn_pool* p);
gdn_status layer_decode(gdn_layer* L, const int32_t* slot_ids, int32_t B, const uint16_t* x,
                        int64_t x_stride, uint16_t* out, int64_t out_stride, void* stream,
                        QPartial* defer, const uint16_t* xsplit = nullptr);

// d: bf16 rows [n, hidden], or null; dp (taken over d when it has slices
// pending): the f32 partials of a deferred projection with N == hidden.
// xsplit (or null; n <= 64): also the 64-column group sums of hn, each split
// exactly into three bf16 parts, [3][64][hidden/64] (hi, mid, lo).
hipError_t launch_add_norm(uint16_t* h, const uint16_t* d, const QPartial* dp, int n, int hidden,
                           const uint16_t* w, float eps, uint16_t* hn, hipStream_t s,
                           uint16_t* xsplit = nullptr);
// h = table[tok[i]] and hn = rms_norm(h) * w in one launch (launch_embed
// followed by launch_add_norm with no addend, bit for bit).
hipError_t launch_embed_norm(const uint16_t* table, const int32_t* tok, int n, int vocab,
                             int hidden, const uint16_t* w, float eps, uint16_t* h, uint16_t* hn,
                             hipStream_t s, uint16_t* xsplit = nullptr);
hipError_t launch_gather_rows(const uint16_t* src, const int32_t* idx, int n, int hidden,
                              uint16_t* dst, hipStream_t s);
// Greedy pick in two passes; pv / pi hold n * argmax_chunks(vocab) partials.
// out_host (or null): a device-mapped pinned host copy of out.
int argmax_chunks(int vocab);
hipError_t launch_argmax(const uint16_t* logits, int64_t ld, int n, int vocab, float* pv, int* pi,
                         int32_t* out, int32_t* out_host, hipStream_t s);

}  // namespace gdn
