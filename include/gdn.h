/*
 * gdn.h -- C ABI of libgdn, the gfx950 (MI355X) GatedDeltaNet decode/prefill
 * path with a device-resident per-sequence state pool.
 *
 * Reference interfaces this ABI replaces (qwen-mlx, Rust + MLX):
 *   - gated_delta_kernel(q,k,v,g,beta,state,T,B,Hk,Hv,Dk,Dv)
 *       src/models/metal_gdn.rs:170-218           -> gdn_recurrent
 *   - compiled_beta_g(b,a,A_log,dt_bias)
 *       src/models/compiled_ops.rs:68-94          -> fused into gdn_decode / gdn_prefill_varlen
 *   - GatedDeltaNet::forward_with_cache, conv/split/norm/gates/recurrence
 *       src/models/qwen3_5.rs:588-658             -> gdn_decode (S=1), gdn_prefill_varlen (S>1)
 *   - Qwen35Executor::stack_caches / unstack_caches
 *       src/scheduler/mlx_executor.rs:42-130      -> the pool itself (slot ids replace copies);
 *                                                    gdn_slots_read / gdn_slots_write keep the
 *                                                    gather / scatter semantics for callers that
 *                                                    need the stacked tensors.
 *   - state init `zeros f32 [B,Hv,Dv,Dk]` / `zeros bf16 [B,3,D]`
 *       src/models/qwen3_5.rs:598-601,613-616,644-648 -> gdn_slots_zero
 *   - error convention of mlx_fast_metal_kernel_apply: 0 = ok, nonzero = failure
 *       src/models/metal_gdn.rs:197-208          -> every function returns gdn_status.
 *
 * Conventions
 *   - All tensors are plain device pointers. bf16 tensors are passed as raw
 *     16-bit patterns (uint16_t). No function allocates caller-visible memory.
 *   - Every compute call is asynchronous on the caller's hipStream_t (passed as
 *     void* so this header needs no HIP include; NULL = the null stream).
 *   - slot_ids are DEVICE int32 arrays. A slot id outside [0, num_slots) makes
 *     the affected work-group skip its sequence entirely (no memory touched) and
 *     latches GDN_FLAG_BAD_SLOT in the pool's device status word, which
 *     gdn_pool_check() reads (synchronously) and clears.
 *   - Slot ids within one call must be distinct: two work-groups updating the
 *     same slot in one launch race. gdn_slots_validate() checks this on demand.
 *     Debug switch: with the library built with -DGDN_DEBUG_SLOTS, or with the
 *     environment variable GDN_DEBUG_SLOTS set to a value other than "0" (read
 *     on every call), gdn_decode*, gdn_recurrent and gdn_prefill_varlen* copy
 *     the slot list to the host, synchronize the stream and return
 *     GDN_ERR_SLOTS for an id out of range or repeated, before any launch.
 *     Off by default: it costs a copy and a host synchronization per call and
 *     breaks HIP graph capture.
 *   - One pool is not reentrant: calls that touch the same slots must be
 *     ordered on one stream by the caller. gdn_prefill_varlen uses a device
 *     workspace held by the pool, so its calls on a pool must be ordered on
 *     one stream; a call that needs more workspace than the pool holds
 *     (it grows with total_tokens, and for a few long sequences also holds
 *     their chunk records) synchronizes its stream and reallocates it, later
 *     calls at or below that size allocate nothing; gdn_pool_reserve sizes it
 *     for any call up to a token count. gdn_decode allocates nothing.
 *   - The decode entries launch kernels only (no memset nodes, no host
 *     synchronisation), so a decode step over every layer can be captured in
 *     one HIP graph and replayed: gdn_decode, gdn_decode_gated, gdn_recurrent,
 *     gdn_slots_zero, gdn_qlinear_forward, and gdn_layer_decode once
 *     gdn_pool_reserve has sized the pool's buffers for the batch.
 *   - Model shape limits: head_k_dim == head_v_dim == 128, conv_kernel == 4,
 *     num_v_heads / num_k_heads in {1, 2, 4}.
 *
 * Tensor layouts (row-major, innermost last)
 *   pool recurrent state, per layer : [num_slots] slots of Hv*Dv*Dk f32. Within a slot,
 *       row dv (Dk contiguous floats, metal_gdn.rs:25-26,149) of value head
 *       hv = hk*R + r (R = Hv/Hk) is item row ir = r*Dv + dv of key head hk,
 *       stored at float offset ((ir/4)*Hk + hk)*4*Dk + (ir%4)*Dk: the Hk
 *       key heads' rows interleave in 4-row (2 KiB) pieces. gdn_slots_read /
 *       gdn_slots_write exchange the reference's [Hv, Dv, Dk] order.
 *   pool conv state, per layer      : [num_slots, K-1, D]   bf16  (qwen3_5.rs:600-604)
 *       D = 2*Hk*Dk + Hv*Dv conv channels, channel order q | k | v (qwen3_5.rs:627-629)
 *   q, k                            : [B, T, Hk, Dk] bf16
 *   v, y                            : [B, T, Hv, Dv] bf16
 *   g (decay multiplier, in (0,1])  : [B, T, Hv] f32
 *   beta                            : [B, T, Hv] bf16
 *   mixed_qkv (pre-conv projection) : [ntok, D] bf16
 *   ab (merged b|a projection)      : [ntok, 2*Hv] bf16, b = ab[:, :Hv], a = ab[:, Hv:]
 *                                     (qwen3_5.rs:583,1037-1040)
 *   A_log, dt_bias                  : [Hv] f32
 *   conv_w (depthwise conv weight)  : [D, K] bf16 (MLX conv1d weight [D,K,1])
 */
#ifndef GDN_H_
#define GDN_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int gdn_status;
#define GDN_OK 0
#define GDN_ERR_INVALID 1     /* bad argument (shape, layer, null pointer)   */
#define GDN_ERR_UNSUPPORTED 2 /* shape outside the compiled kernel family     */
#define GDN_ERR_HIP 3         /* HIP runtime error (launch, memcpy, ...)      */
#define GDN_ERR_OOM 4         /* device allocation failed                     */
#define GDN_ERR_SLOTS 5       /* slot ids failed validation                   */

/* Device status bits latched by kernels (gdn_pool_check). */
#define GDN_FLAG_BAD_SLOT 0x1u      /* a slot id was outside [0, num_slots)      */
#define GDN_FLAG_DUP_SLOT 0x2u      /* gdn_slots_validate found a repeated id    */
#define GDN_FLAG_BAD_SEQLENS 0x4u   /* cu_seqlens not non-decreasing / too long  */

#define GDN_ALL_LAYERS (-1)

typedef struct gdn_pool gdn_pool;

typedef struct gdn_pool_desc {
  int32_t num_layers;  /* GDN layers held by the pool (30 for Qwen3.5-35B-A3B) */
  int32_t num_slots;   /* sequence slots per layer                            */
  int32_t num_k_heads; /* Hk  (linear_num_key_heads)                          */
  int32_t num_v_heads; /* Hv  (linear_num_value_heads)                        */
  int32_t head_k_dim;  /* Dk  (linear_key_head_dim), must be 128              */
  int32_t head_v_dim;  /* Dv  (linear_value_head_dim), must be 128            */
  int32_t conv_kernel; /* K   (linear_conv_kernel_dim), must be 4             */
  int32_t device;      /* HIP device ordinal the pool lives on                */
} gdn_pool_desc;

/* Thread-local message describing the last non-OK status on this thread. */
const char* gdn_last_error(void);

/* Library version string ("gdn <major>.<minor> gfx950"). */
const char* gdn_version(void);

/* Allocate and zero a pool: per layer, num_slots x Hv*Dv*Dk f32 recurrent
 * state and [num_slots,K-1,D] bf16 conv state (both start at +0.0). */
gdn_status gdn_pool_create(const gdn_pool_desc* desc, gdn_pool** out);
gdn_status gdn_pool_destroy(gdn_pool* pool);
/* The pool's descriptor as created. */
gdn_status gdn_pool_describe(const gdn_pool* pool, gdn_pool_desc* desc);

/* Device pointers of one layer's state arrays (for inspection / export). */
gdn_status gdn_pool_layer_state(gdn_pool* pool, int32_t layer, float** state,
                                uint16_t** conv_state);

/* Sizes in bytes of one slot's recurrent and conv state in one layer. */
gdn_status gdn_pool_slot_bytes(const gdn_pool* pool, size_t* state_bytes,
                               size_t* conv_bytes);

/* Read (and clear) the pool's latched device status flags. Synchronises the
 * given stream first. */
gdn_status gdn_pool_check(gdn_pool* pool, void* stream, uint32_t* flags);

/* Host-side slot allocator (free list, lowest id first). Replaces the
 * reference's per-sequence `Qwen35State` arrays (mlx_executor.rs:19-21):
 * one slot id addresses the sequence's state in every layer. */
gdn_status gdn_slot_alloc(gdn_pool* pool, int32_t* slot);
gdn_status gdn_slot_free(gdn_pool* pool, int32_t slot);
gdn_status gdn_slots_in_use(const gdn_pool* pool, int32_t* count);

/* Zero the recurrent and conv state of n slots in `layer` (or every layer
 * with GDN_ALL_LAYERS). Replaces the missing-cache zero init of
 * qwen3_5.rs:598-601,613-616,644-648. Uses a fill kernel (no memset node), so
 * it may be captured in a HIP graph. */
gdn_status gdn_slots_zero(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                          int32_t n, void* stream);

/* Gather n slots of `layer` into caller buffers (stack_caches,
 * mlx_executor.rs:92-115): state_out [n,Hv,Dv,Dk] f32, conv_out [n,K-1,D] bf16.
 * Either output may be NULL. Bit-exact copies. */
gdn_status gdn_slots_read(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                          int32_t n, float* state_out, uint16_t* conv_out,
                          void* stream);

/* Scatter caller buffers into n slots (unstack_caches, mlx_executor.rs:118-130).
 * Either input may be NULL. Bit-exact copies. */
gdn_status gdn_slots_write(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                           int32_t n, const float* state_in, const uint16_t* conv_in,
                           void* stream);

/* Device-side check of a slot-id list: range and uniqueness. Latches
 * GDN_FLAG_BAD_SLOT / GDN_FLAG_DUP_SLOT (read them with gdn_pool_check). */
gdn_status gdn_slots_validate(gdn_pool* pool, const int32_t* slot_ids, int32_t n,
                              void* stream);

/* The gated delta rule recurrence on already-prepared q/k/v/g/beta, state in
 * pool slots, updated in place. Same arithmetic as gated_delta_kernel
 * (metal_gdn.rs:10-67,170-218): per t, s *= g; kv = s.k; d = (v-kv)*beta;
 * s += k*d; y = s.q. q and k are used as given (the caller normalises them).
 * B sequences x T tokens each; slot_ids[B]. */
gdn_status gdn_recurrent(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                         int32_t B, int32_t T, const uint16_t* q, const uint16_t* k,
                         const uint16_t* v, const float* g, const uint16_t* beta,
                         uint16_t* y, void* stream);

/* Fused S=1 decode step of one GDN layer for B sequences (qwen3_5.rs:593-610,
 * 626-658 + compiled_ops.rs:30-43), in one launch:
 *   conv window [state | x] . w  -> silu -> split q|k|v -> q,k rms-norm with the
 *   baked weights bf16(1/Dk), bf16(1/sqrt(Dk)), eps 1e-6 -> beta = sigmoid(b),
 *   g = exp(-exp(A_log) * log(exp(a+dt_bias)+1)) -> recurrence -> y.
 * The rolling conv state and the recurrent state of each slot are updated in
 * place. mixed_qkv [B,D], ab [B,2Hv], y [B,Hv,Dv]; B <= num_slots. */
gdn_status gdn_decode(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                      int32_t B, const uint16_t* mixed_qkv, const uint16_t* ab,
                      const float* A_log, const float* dt_bias,
                      const uint16_t* conv_w, uint16_t* y, void* stream);

/* gdn_decode with the RMSNormGated epilogue fused into the readout
 * (qwen3_5.rs:660-665, norm_gate_fn in compiled_ops.rs:247-263): per
 * (sequence, value head), out = silu(z) * rms_norm(y, norm_w, norm_eps) over
 * the Dv outputs of the recurrence, each elementwise op rounded to bf16. It
 * reads the merged projection rows as the reference produces them
 * (qwen3_5.rs:572-577): qkvz [B, row_stride] bf16 holds q|k|v in columns
 * [0, D) and z in columns [D, D + Hv*Dv), row_stride >= D + Hv*Dv, so no copy
 * of either part is needed; ab [B, ab_stride] holds b|a in its first 2*Hv
 * columns (ab_stride >= 2*Hv; a view into a merged projection output works as
 * the reference's ab slices do, qwen3_5.rs:580-584). norm_w [Dv] bf16 (the layer's norm.weight),
 * norm_eps the model's rms_norm_eps. out [B, Hv, Dv] bf16 is the out_proj
 * input; y [B, Hv, Dv] (the ungated recurrence output) may be NULL. Same state
 * updates as gdn_decode. */
gdn_status gdn_decode_gated(gdn_pool* pool, int32_t layer, const int32_t* slot_ids, int32_t B,
                            const uint16_t* qkvz, int64_t row_stride, const uint16_t* ab,
                            int64_t ab_stride, const float* A_log, const float* dt_bias,
                            const uint16_t* conv_w, const uint16_t* norm_w, float norm_eps,
                            uint16_t* out, uint16_t* y, void* stream);

/* Varlen prefill of nseq sequences packed along the token axis
 * (qwen3_5.rs:611-658 with S>1; the reference runs them one at a time, B=1):
 * sequence i owns tokens [cu_seqlens[i], cu_seqlens[i+1]) of mixed_qkv / ab / y
 * and slot slot_ids[i]. Each sequence starts from its slot's current conv and
 * recurrent state (zero after gdn_slots_zero, as the reference's fresh
 * prefill) and leaves its final states there. cu_seqlens is a DEVICE int32
 * array of nseq+1 entries with cu_seqlens[0] == 0 and
 * cu_seqlens[nseq] == total_tokens <= 4,194,240 (65535 tiles of 64 tokens);
 * a cu_seqlens that breaks these latches GDN_FLAG_BAD_SEQLENS (the kernels
 * clamp every bound they read). Uses the chunked (WY form, chunk 64)
 * algorithm; results equal the token-by-token recurrence within f32/bf16
 * rounding. Two schedules give the same bits: one work-group per (sequence,
 * value head), or, for a few long sequences (at most 96 sequence-heads, 1024
 * tokens per sequence on average, 262,144 tokens per call), the chunks'
 * state-independent blocks formed for all chunks at once and 2 or 4
 * work-groups per (sequence, value head). The environment variable
 * GDN_PREFILL_WAVES = 8 (the first), 4 or 2 (the second) forces one.
 * The second schedule, with at least 8,192 tokens in the call and at most
 * half as many work-groups as the device has CUs (one 16,384-token prompt at
 * 32 value heads: 128), runs as a pipeline of 2 to 8 token segments (each
 * twice the one before): the next
 * segment's conv/norm and block-forming kernels go to a second stream that
 * the pool makes on first use and keeps (default priority, non-blocking),
 * beside the state products of the segment before on `stream`. The call is
 * still ordered on `stream` alone (it starts after the work already queued
 * there, and what is queued there after it waits for all of it) and gives the
 * same bits as one pass. Not under stream capture, nor in
 * gdn_prefill_varlen_noalloc; GDN_PREFILL_SEGMENTS = n forces n segments (1:
 * one pass). */
gdn_status gdn_prefill_varlen(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                              const int32_t* cu_seqlens, int32_t nseq,
                              int32_t total_tokens, const uint16_t* mixed_qkv,
                              const uint16_t* ab, const float* A_log,
                              const float* dt_bias, const uint16_t* conv_w,
                              uint16_t* y, void* stream);

/* gdn_prefill_varlen for callers that cannot allocate device memory (code
 * under HIP graph capture, serving loops that forbid hipMalloc). No
 * counterpart in the reference. Same arguments and results; the workspace
 * is a fixed 64 MiB array per device held by the library until the process
 * ends, instead of the pool's grown buffer. The call takes the schedule
 * gdn_prefill_varlen would take when that schedule's workspace fits, else
 * the one-group-per-head schedule (both give the same bits). A call whose
 * workspace on that schedule (16,576 bytes per token at 16 key / 32 value
 * heads: up to 4,048 tokens) exceeds the array fails with GDN_ERR_INVALID
 * before any launch. Allocates nothing
 * (hipMalloc, hipFree or otherwise). Every call on a device shares that
 * array: calls that overlap on one device race, so order them on one stream. */
gdn_status gdn_prefill_varlen_noalloc(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                                      const int32_t* cu_seqlens, int32_t nseq,
                                      int32_t total_tokens, const uint16_t* mixed_qkv,
                                      const uint16_t* ab, const float* A_log,
                                      const float* dt_bias, const uint16_t* conv_w,
                                      uint16_t* y, void* stream);

/* gdn_prefill_varlen on merged projection rows with the RMSNormGated epilogue
 * fused into the chunk kernel's readout (qwen3_5.rs:660-665 after the S>1
 * path): out [total_tokens, Hv, Dv] = silu(z) * rms_norm(y, norm_w, norm_eps)
 * per (token, value head). qkvz [total_tokens, row_stride] holds q|k|v in
 * columns [0, D) and z in [D, D + Hv*Dv) (row_stride >= D + Hv*Dv, a multiple
 * of 8, qkvz 16-byte aligned); ab [total_tokens, ab_stride] holds b|a in its
 * first 2*Hv columns. y [total_tokens, Hv, Dv] (the ungated output) may be
 * NULL. Same state updates as gdn_prefill_varlen. */
gdn_status gdn_prefill_varlen_gated(gdn_pool* pool, int32_t layer, const int32_t* slot_ids,
                                    const int32_t* cu_seqlens, int32_t nseq, int32_t total_tokens,
                                    const uint16_t* qkvz, int64_t row_stride, const uint16_t* ab,
                                    int64_t ab_stride, const float* A_log, const float* dt_bias,
                                    const uint16_t* conv_w, const uint16_t* norm_w,
                                    float norm_eps, uint16_t* out, uint16_t* y, void* stream);

/* ------------------------------------------------------------------------
 * 4-bit affine-quantized linear layer: the GDN block's input projections.
 *
 * Replaces mlx_rs::ops::quantized_matmul(x, w, scales, biases, transpose=true,
 * group_size=64, bits=4) on the merged projection weights
 * (qwen3_5.rs:572-586), including the load-time merge of the parts along the
 * output axis (qwen3_5.rs:1023-1053: qkv|z into merged_qkvz, b|a into
 * merged_ab). Weight format as MLX stores it: w uint32 [N_i, K/8] with element
 * k of row n in bits 4*(k%8) of word k/8; scales, biases bf16 [N_i, K/64];
 * dequantized weight = scales * q + biases.
 *
 * y[m, n] = sum_k x[m, k] * w[n, k], computed exactly up to f32 accumulation
 * and rounded once to bf16.
 * ------------------------------------------------------------------------ */
typedef struct gdn_qlinear gdn_qlinear;

/* Merge nparts MLX-format parts (device pointers, part i has part_rows[i]
 * output rows) into one layer with N = sum(part_rows) outputs and repack it
 * for the kernel on `device`. The layer owns its memory (about N*K/2 +
 * 3*N*K/32 bytes, plus K/512 * 64 * N f32 partial sums for layers whose
 * decode-sized calls split K: K > 2048, or N < 8192 with K >= 1024); the
 * sources are only read, and may be freed once this returns (it synchronises
 * `stream`). Supported: bits 4, group_size 64, K a multiple of 512 up to
 * 4096, part_rows multiples of 16. */
gdn_status gdn_qlinear_create(int32_t K, int32_t nparts, const int32_t* part_rows,
                              const uint32_t* const* w, const uint16_t* const* scales,
                              const uint16_t* const* biases, int32_t group_size, int32_t bits,
                              int32_t device, void* stream, gdn_qlinear** out);
gdn_status gdn_qlinear_destroy(gdn_qlinear* layer);

/* Input width K and output width N of a layer. */
gdn_status gdn_qlinear_dims(const gdn_qlinear* layer, int32_t* K, int32_t* N);

/* y [M, y_stride] bf16 = x [M, x_stride] bf16 . W^T over the first N columns
 * (columns past N untouched). x: 16-byte aligned, x_stride >= K and a
 * multiple of 8; y: 8-byte aligned, y_stride >= N and a multiple of 4;
 * M <= 8,388,480. Allocates nothing. Calls on one layer must be ordered on
 * one stream (a K-split call uses the layer's partial-sum buffer). For the
 * merged qkv|z|b|a layer the
 * output row is [q|k|v|z|b|a], which gdn_decode_gated reads in place
 * (qkvz = y, row_stride = y_stride; ab = y + D + Hv*Dv, ab_stride = y_stride). */
gdn_status gdn_qlinear_forward(const gdn_qlinear* layer, const uint16_t* x, int64_t x_stride,
                               int32_t M, uint16_t* y, int64_t y_stride, void* stream);

/* Residual add and RMSNorm of n hidden-size rows: the decoder layer's seam
 * around each mixer (qwen3_5.rs:729-739: h = h + mixer output, then
 * input_layernorm / post_attention_layernorm, an RMSNorm with weight w):
 *   h  <- bf16(h + d)                       (skipped when d is NULL)
 *   hn  = bf16(w * bf16(h * r)),  r = 1 / sqrt(mean(h^2) + eps)
 * group_sums (or NULL; needs n <= 64 and hidden % 64 == 0): the 64-column
 * group sums of each hn row, each split exactly into three bf16 parts,
 * [3][64][hidden/64] (hi, mid, lo; rows n..63 untouched), the operand of
 * gdn_qlinear_forward_sums. hidden <= 4096 and a multiple of 8; h, d, hn and
 * w 16-byte aligned. Runs on the current device. */
gdn_status gdn_add_rms_norm(uint16_t* h, const uint16_t* d, int32_t n, int32_t hidden,
                            const uint16_t* w, float eps, uint16_t* hn, uint16_t* group_sums,
                            void* stream);

/* gdn_qlinear_forward on rows x whose 64-column group sums a producer has
 * already formed (gdn_add_rms_norm's group_sums of the same rows). The
 * decode-sized paths (M <= 64) of a K = 2048 layer that runs whole-K tiles
 * and of every layer at least 131,072 columns wide (lm_head) take the sums
 * instead of forming them with products of x; every other shape ignores
 * group_sums. Rows M..63 of group_sums are read but only reach outputs past
 * row M, which are not written. Same arguments and results contract as
 * gdn_qlinear_forward otherwise. It has no counterpart in the reference,
 * whose quantized_matmul (qwen3_5.rs:572-586) forms the sums itself; it is
 * the fused norm-to-projection hand-off the executor uses for in_proj and
 * lm_head. */
gdn_status gdn_qlinear_forward_sums(const gdn_qlinear* layer, const uint16_t* x, int64_t x_stride,
                                    const uint16_t* group_sums, int32_t M, uint16_t* y,
                                    int64_t y_stride, void* stream);

/* ------------------------------------------------------------------------
 * One GatedDeltaNet layer end to end: GatedDeltaNet::forward_with_cache
 * (qwen3_5.rs:558-668) with the (conv_state, recurrent_state) cache pair
 * replaced by pool slots:
 *   proj = in_proj(x)                          [q|k|v|z|b|a], one gdn_qlinear_forward
 *   gated = gdn_decode_gated / gdn_prefill_varlen_gated on column views of proj
 *   out = out_proj(gated)                      one gdn_qlinear_forward
 * x and out are hidden-size bf16 rows (the decoder layer's input_layernorm
 * output and the mixer output the residual adds, qwen3_5.rs:729-739).
 * The layer keeps pointers only: the pool, the two projections and the
 * weight tensors must outlive it. Activations go to a buffer held by the
 * pool (shared by every layer of the pool, so the pool's calls are ordered
 * on one stream): a call needing more of it than any earlier call
 * synchronises its stream and grows it; gdn_pool_reserve sizes it (and the
 * prefill workspace, for either prefill schedule, also one forced with the
 * environment variable GDN_PREFILL_WAVES) up front so later calls allocate
 * nothing. A pool driven by an executor belongs to it: other calls on the
 * pool must be ordered after the executor's work (its stream, or a
 * synchronisation). Growing the activation buffer makes the executor drop
 * and capture anew the step graphs that held the old one.
 * ------------------------------------------------------------------------ */
typedef struct gdn_layer gdn_layer;

typedef struct gdn_layer_desc {
  gdn_pool* pool;
  int32_t layer;                /* this layer's state arrays in the pool      */
  const gdn_qlinear* in_proj;   /* merged q|k|v|z|b|a: N = D + Hv*Dv + 2*Hv,
                                   K = hidden size (qwen3_5.rs:1037-1053)     */
  const gdn_qlinear* out_proj;  /* Hv*Dv -> hidden size (qwen3_5.rs:668)     */
  const float* A_log;           /* [Hv] f32                                   */
  const float* dt_bias;         /* [Hv] f32                                   */
  const uint16_t* conv_w;       /* [D, K] bf16, 8-byte aligned                */
  const uint16_t* norm_w;       /* [Dv] bf16 (linear_attn.norm.weight)        */
  float norm_eps;               /* rms_norm_eps                               */
} gdn_layer_desc;

gdn_status gdn_layer_create(const gdn_layer_desc* desc, gdn_layer** out);
gdn_status gdn_layer_destroy(gdn_layer* layer);

/* Size the pool's activation buffer and prefill workspace for calls of up
 * to max_tokens tokens (decode batch size or packed prefill tokens), the
 * chunk records of the few-long-sequences schedule included. */
gdn_status gdn_pool_reserve(gdn_pool* pool, int32_t max_tokens, void* stream);

/* S = 1 step of B sequences: x [B, x_stride] -> out [B, out_stride], state of
 * slot_ids[B] updated in place. x: 16-byte aligned, x_stride a multiple of 8;
 * out: 8-byte aligned, out_stride a multiple of 4; both strides >= hidden. */
gdn_status gdn_layer_decode(gdn_layer* layer, const int32_t* slot_ids, int32_t B,
                            const uint16_t* x, int64_t x_stride, uint16_t* out,
                            int64_t out_stride, void* stream);

/* Varlen prefill of nseq packed sequences (cu_seqlens as gdn_prefill_varlen):
 * x [total_tokens, x_stride] -> out [total_tokens, out_stride]. */
gdn_status gdn_layer_prefill(gdn_layer* layer, const int32_t* slot_ids,
                             const int32_t* cu_seqlens, int32_t nseq, int32_t total_tokens,
                             const uint16_t* x, int64_t x_stride, uint16_t* out,
                             int64_t out_stride, void* stream);

/* ------------------------------------------------------------------------
 * Executor: the ModelExecutor contract (src/scheduler/executor.rs:21-49) on
 * pool slots, in place of Qwen35Executor (src/scheduler/mlx_executor.rs:23-257).
 * A sequence's per-layer caches (Qwen35State, mlx_executor.rs:19-21) are one
 * slot id, the same in every layer, so stack_caches / unstack_caches
 * (:92-130) disappear: a decode step hands the layers B slot ids. Prefill
 * admits the sequence (slot alloc + zero in every layer: the fresh caches of
 * qwen3_5.rs:598-648), gdn_exec_release retires it (the Sequence's state
 * dropped), submit / collect pipeline one batch against the host
 * (mlx_executor.rs:195-254 as driven by qwen_mlx_serve.rs:110-177).
 *
 * The model the executor runs is the Qwen3.5 decoder stack without its MLPs:
 *   h = embed[token]; per layer l: h = h + mixer_l(rms_norm(h, input_norm_w[l]));
 *   token = argmax(lm_head(rms_norm(h, final_norm_w)))
 * (Qwen35Model::forward, qwen3_5.rs:826-880; DecoderLayer::forward_with_cache
 * :723-743 without the MLP half). A mixer is a GatedDeltaNet layer or, at the
 * positions attn_layers name, an attention layer (qwen3_5.rs:377-455: merged
 * q|k|v projection, gdn_attn_forward on the executor's gdn_kv, o_proj). The
 * KV cache uses the pool's slot ids. MoE MLPs and temperature sampling are
 * outside this library; the greedy pick keeps runs reproducible.
 *
 * One thread owns an executor (qwen_mlx_serve.rs:96-99). All its device work
 * runs on the stream given at creation, in call order. Sequence ids are the
 * caller's (SequenceId, sequence.rs:7); token ids are checked against the
 * vocabulary on the host.
 * ------------------------------------------------------------------------ */
typedef struct gdn_exec gdn_exec;
typedef struct gdn_kv gdn_kv;

/* One attention layer of the stack (Qwen35Attention, qwen3_5.rs:377-455). */
typedef struct gdn_exec_attn_layer {
  int32_t position;              /* index in the decoder stack                      */
  const gdn_qlinear* qkv_proj;   /* hidden -> Hq*512 + 2*Hkv*256: per query head 256
                                    query then 256 gate outputs, then k, then v   */
  const gdn_qlinear* o_proj;     /* Hq*256 -> hidden                                */
  const uint16_t* q_norm_w;      /* [256] bf16                                      */
  const uint16_t* k_norm_w;      /* [256] bf16                                      */
} gdn_exec_attn_layer;

typedef struct gdn_exec_desc {
  gdn_pool* pool;                       /* every sequence's GDN state, one slot each     */
  int32_t num_layers;
  gdn_layer* const* layers;             /* the GDN layers in model order (on `pool`)     */
  const uint16_t* const* input_norm_w;  /* per decoder layer, GDN and attention, in stack
                                           order: [hidden] bf16 input_layernorm         */
  const uint16_t* final_norm_w;         /* [hidden] bf16                                 */
  float rms_eps;
  const uint16_t* embed;                /* [vocab, hidden] bf16, 16-byte aligned         */
  const gdn_qlinear* head;              /* lm_head: hidden -> vocab (sets both sizes)    */
  int32_t max_batch;                    /* decode batch bound (max_batch_size)           */
  int32_t max_prompt;                   /* longest prompt one prefill takes              */
  int32_t device;                       /* HIP device of the pool and weights            */
  /* attention layers: num_attn_layers = 0 for a GDN-only stack */
  int32_t num_attn_layers;
  const gdn_exec_attn_layer* attn_layers; /* increasing positions; attention layer i uses
                                           kv layer i                                  */
  gdn_kv* kv;                           /* num_slots >= the pool's, max_step_tokens >=
                                           max(max_batch, max_prompt)                   */
  float rope_theta;
  int32_t rotary_dim;
} gdn_exec_desc;

/* Allocates the executor's buffers (activations for max(max_batch,
 * max_prompt) rows, logits for max_batch rows, pinned staging) and sizes the
 * pool's layer buffers with gdn_pool_reserve: later decode steps allocate
 * nothing. A prefill on a stack with attention layers may grow the KV cache's
 * attention workspace (see gdn_kv_step). max_prompt must fit one slot's KV
 * pages (max_pages_per_slot * 64 tokens). */
gdn_status gdn_exec_create(const gdn_exec_desc* desc, void* stream, gdn_exec** out);
/* Waits for the stream, frees the buffers and the slots still held. */
gdn_status gdn_exec_destroy(gdn_exec* exec);

/* ModelExecutor::prefill (executor.rs:23): admit seq_id (a free slot, or its
 * own slot again if it is known) with zeroed state, run the prompt through
 * every layer and return the first picked token. Synchronous. Checks that
 * fail before admission change nothing; a failure after it retires every
 * sequence of the call (slot and KV pages freed, id forgotten: a known
 * sequence has given back its pages and its state is no longer usable), and
 * the caller prefills them again. */
gdn_status gdn_exec_prefill(gdn_exec* exec, uint64_t seq_id, const int32_t* prompt, int32_t len,
                            uint32_t* first_token);

/* Prefill of nseq <= max_batch distinct sequences in one pass: the prompts are
 * packed back to back in `prompts` (lens[i] >= 1 tokens each, at most
 * max_prompt in total) and share every layer's varlen prefill launches
 * (the reference prefills one sequence per call, scheduler.rs:196-216).
 * first_tokens[i] is sequence i's first picked token. The projections' row
 * count changes with the packing, and with it their f32 summation order, so
 * results equal separate prefills up to that rounding. A call that finds no
 * free slot for some sequence admits none of its new sequences. */
gdn_status gdn_exec_prefill_batch(gdn_exec* exec, int32_t nseq, const uint64_t* seq_ids,
                                  const int32_t* prompts, const int32_t* lens,
                                  uint32_t* first_tokens);

/* ModelExecutor::decode_batch (executor.rs:26): one token for each of B
 * prefilled, distinct sequences, fed their current tokens; the results in
 * input order. = submit_batch + collect_batch. */
gdn_status gdn_exec_decode_batch(gdn_exec* exec, const uint64_t* seq_ids, const uint32_t* tokens,
                                 int32_t B, uint32_t* next_tokens);

/* ModelExecutor::submit_batch / collect_batch (executor.rs:31-42): queue the
 * step and return at once; collect waits for it. A submit with a step still
 * uncollected fails (gdn_exec_submit_next below may queue a second one). A
 * prefill between the two is allowed (it waits for the batch).
 * A decode step replays HIP graphs: the first step at a batch size B
 * captures the step's launches (on a private stream) as one graph per span
 * between attention calls, which run eagerly because their launch shape
 * follows the step's KV plan; later steps at B launch the graphs on the
 * executor's stream. Results are bit-identical to launching kernel by kernel,
 * which the environment variable GDN_EXEC_GRAPHS=0 (read at gdn_exec_create)
 * selects. A batch size whose capture fails runs eagerly. A GDN layer's
 * in_proj and lm_head take their rows' group sums from the preceding norm
 * (gdn_add_rms_norm / gdn_qlinear_forward_sums) when B <= 64; the variable
 * GDN_EXEC_SPLIT_SUMS=0 (read at gdn_exec_create) makes them form them
 * themselves. */
gdn_status gdn_exec_submit_batch(gdn_exec* exec, const uint64_t* seq_ids, const uint32_t* tokens,
                                 int32_t B);
/* Collects the oldest uncollected step (of at most two, see below). */
gdn_status gdn_exec_collect_batch(gdn_exec* exec, uint32_t* next_tokens, int32_t B);

/* The double-buffered decode of src/bin/qwen_mlx_infer.rs:136-187 (step N+1
 * built on step N's unevaluated token array, then async-evaluated before
 * step N is read): queue one more decode step for the sequences of the last
 * submitted step, in the same order, each fed the token that step picks, read
 * on the device (no host round trip). The step may be uncollected: then two
 * are, and collect_batch returns them oldest first. B must be that step's B.
 * Fails (queueing nothing) with nothing to follow -- no step submitted since
 * the executor was created or since the last prefill or release -- and with
 * two steps uncollected. Tokens are those of submit_batch fed the collected
 * picks, bit for bit. */
gdn_status gdn_exec_submit_next(gdn_exec* exec, int32_t B);

/* The sequence is finished (its Sequence and state dropped): its slot goes
 * back to the pool. Work already queued on the slot still completes first. */
gdn_status gdn_exec_release(gdn_exec* exec, uint64_t seq_id);

/* ModelExecutor::max_batch_size / supports_pipeline (executor.rs:45-48). */
int32_t gdn_exec_max_batch_size(const gdn_exec* exec);
int32_t gdn_exec_supports_pipeline(const gdn_exec* exec);

/* Introspection: the slot of a sequence; the device logits of the last
 * forward (rows x vocab bf16, valid until the next call). */
gdn_status gdn_exec_seq_slot(const gdn_exec* exec, uint64_t seq_id, int32_t* slot);
gdn_status gdn_exec_logits(const gdn_exec* exec, const uint16_t** logits, int32_t* rows,
                           int32_t* vocab);

/* ------------------------------------------------------------------------
 * Attention layers: paged KV cache and the attention step
 * (Qwen35Attention::forward_with_cache, qwen3_5.rs:377-455).
 *
 * The reference grows one [1, Hkv, len, 256] key and value array per
 * sequence and layer by concatenation (qwen3_5.rs:419-424) and batches them
 * by zero-padding to the longest (mlx_executor.rs:57-88); its decode
 * attention then has no mask and its RoPE one offset for the whole batch
 * (qwen3_5.rs:410,443-447), so with B > 1 shorter sequences attend to padding
 * at wrong positions. Here the cache is pages of 64 tokens (a page id covers
 * the same positions in every layer), each sequence slot has a page table,
 * and every token carries its own position: keys are masked at the
 * sequence's length and RoPE uses the token's position.
 *
 * A step: gdn_kv_step plans the tokens appended for n sequences (they are
 * packed in that order, ntok[i] rows each, in every tensor below), then each
 * attention layer calls gdn_attn_forward on those rows, on the same stream.
 * Per token: rms-norm of q and k with their weights, rotate-half RoPE over the
 * first rotary_dim dimensions at the token's position (base rope_theta), K/V
 * appended to the cache, causal attention over the sequence's cached keys
 * (scale 1/sqrt(256)), out = attn * sigmoid(gate) per head. Head dim 256;
 * num_q_heads / num_kv_heads = 4 or 8. Results are deterministic for a given
 * step; the same tokens in a step with other sequences may differ by one bf16
 * ulp (the step's key blocks are split evenly over the workers, so a token's
 * partial sums depend on the whole step).
 * ------------------------------------------------------------------------ */
typedef struct gdn_kv_desc {
  int32_t num_layers;          /* attention layers                               */
  int32_t num_slots;           /* sequences the cache can hold                   */
  int32_t num_pages;           /* 64-token pages shared by all slots             */
  int32_t max_pages_per_slot;  /* longest context / 64                           */
  int32_t num_q_heads;         /* num_attention_heads                            */
  int32_t num_kv_heads;        /* num_key_value_heads                            */
  int32_t head_dim;            /* must be 256                                    */
  int32_t max_step_tokens;     /* most tokens one step appends (all sequences)   */
  int32_t device;
  int32_t max_workers;         /* waves a step's attention is split over; 0 =
                                  1024 when each key is read about once (decode
                                  steps), 2048 when a step re-reads its keys
                                  (prompts); fewer when sharing the GPU        */
} gdn_kv_desc;

/* Per layer num_pages x 128 KiB of bf16 K/V (at 2 kv heads), a page table,
 * and staging for max_step_tokens tokens. */
gdn_status gdn_kv_create(const gdn_kv_desc* desc, gdn_kv** out);
gdn_status gdn_kv_destroy(gdn_kv* kv);
/* The cache's descriptor as created (max_workers as given). */
gdn_status gdn_kv_describe(const gdn_kv* kv, gdn_kv_desc* desc);

/* A sequence leaves (or starts over): its pages go back to the free list. */
gdn_status gdn_kv_release(gdn_kv* kv, int32_t slot);
gdn_status gdn_kv_length(const gdn_kv* kv, int32_t slot, int64_t* len);
gdn_status gdn_kv_free_pages(const gdn_kv* kv, int32_t* count);

/* Plan one step: sequence slots[i] (HOST array, distinct) appends ntok[i] >= 1
 * tokens at positions len .. len + ntok[i] - 1, taking pages from the free
 * list; the per-token metadata is copied to the device on `stream`. Fails
 * (changing nothing) when pages, max_pages_per_slot or max_step_tokens do not
 * suffice. A step with one token per sequence is a decode step, a prompt is
 * one sequence's ntok tokens. gdn_kv_create sizes the attention workspace for
 * every decode step; a step with prompts whose schedule needs more grows it
 * here (waiting for `stream` first). */
gdn_status gdn_kv_step(gdn_kv* kv, int32_t n, const int32_t* slots, const int32_t* ntok,
                       void* stream);

/* One attention layer on the planned step's T packed tokens: q_full [T,
 * q_stride] (per query head 256 query then 256 gate values, the q_proj output
 * of qwen3_5.rs:385-389), k, v [T, stride] (Hkv x 256 each), q_norm_w /
 * k_norm_w [256] bf16; out [T, out_stride] (Hq x 256 gated rows, the o_proj
 * input). */
gdn_status gdn_attn_forward(gdn_kv* kv, int32_t layer, const uint16_t* q_full, int64_t q_stride,
                            const uint16_t* k, int64_t k_stride, const uint16_t* v,
                            int64_t v_stride, const uint16_t* q_norm_w, const uint16_t* k_norm_w,
                            float norm_eps, float rope_theta, int32_t rotary_dim, uint16_t* out,
                            int64_t out_stride, void* stream);

/* Copy a slot's cached keys and values of one layer (rows after norm and
 * RoPE, as attention reads them) into k_out / v_out [Hkv, len, 256] bf16 (either
 * may be NULL). For export and inspection. */
gdn_status gdn_kv_read(gdn_kv* kv, int32_t layer, int32_t slot, uint16_t* k_out, uint16_t* v_out,
                       void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN_H_ */
