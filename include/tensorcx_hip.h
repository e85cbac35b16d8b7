/*
 * tensorcx_hip.h: C ABI of the MI355X (gfx950) hip device for tensor.cx.
 *
 * The C++ `tensorcx::hip::HipBackend` (tensor.cx_amd/cpp/tensorcx/backends/hip)
 * implements the reference's backend interface `Backend::execute`
 * (reference cpp/tensorcx/core/backend.h:67-73) on top of these entry points,
 * exactly where the reference's CUDA prototype calls the CUDA runtime and its
 * `launch_*` kernel wrappers. Every entry point takes plain pointers, sizes and
 * POD descriptors, returns a status code with the values of
 * `tensorcx::StatusCode` (reference core/status.h:8-13), never throws, and
 * leaves a message for `tcx_hip_last_error()` on failure. Kernel launchers
 * enqueue on the given stream and never allocate: scratch space comes in
 * through a workspace argument sized by the matching *_workspace_bytes query.
 */
#ifndef TENSORCX_HIP_H_
#define TENSORCX_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Values of tensorcx::StatusCode (reference core/status.h:8-13). */
#define TCX_OK 0
#define TCX_INVALID_ARGUMENT 1
#define TCX_UNAVAILABLE 2
#define TCX_INTERNAL 3

/* Values of tensorcx::DType (reference core/dtype.h:8-12). */
#define TCX_FLOAT32 0
#define TCX_INT32 1
#define TCX_BOOL 2 /* 1-byte bool (fill and attention masks) */

typedef void* tcx_stream_t; /* a hipStream_t */

/* ------------------------------------------------------------------ runtime */

/* Message of the last failed call on this thread ("" if none). */
const char* tcx_hip_last_error(void);

/* Initialises the HIP runtime once per process and checks for a device.
 * Replaces cuda::available() (reference backends/cuda/cuda_backend.h:37;
 * cuda_backend.cpp:166-169). Returns TCX_UNAVAILABLE without a device, and in
 * any process forked from the one that loaded the library, before any HIP
 * call there (cf. cuda_context.cpp:16-20). Every entry point that reaches the
 * runtime checks this first. */
int tcx_hip_init(void);
int tcx_hip_device_count(int* count);

typedef struct {
  char name[256];
  char arch[64];            /* gcnArchName, e.g. "gfx950:sramecc+:xnack-" */
  int compute_units;
  int clock_khz;
  int memory_clock_khz;
  int memory_bus_width;
  int l2_bytes;
  int runtime_version;
  int driver_version;
  size_t total_bytes;
  size_t free_bytes;
} tcx_hip_device_info_t;

/* Replaces cuda::device_name()/device_info() (cuda_backend.h:38-44). */
int tcx_hip_device_info(int device, tcx_hip_device_info_t* info);

/* This thread's stream (created on first use, default priority). Every
 * HipBackend::execute runs on it and synchronises it before returning, the
 * reference's synchronous completion contract (docs/BACKENDS.md:73-80). */
int tcx_hip_stream(tcx_stream_t* stream);
int tcx_hip_stream_synchronize(tcx_stream_t stream);

/* ------------------------------------------------------------------- memory */

typedef struct tcx_hip_pool tcx_hip_pool_t;

/* Device allocation for a tensor buffer: from this thread's active pool when
 * one is entered, else hipMalloc. *owner receives the pool the block came from
 * (or NULL) and must be passed back to tcx_hip_release. Replaces
 * CudaBuffer::create (cuda_backend.cpp:58-85). Zero bytes yields NULL. */
int tcx_hip_allocate(size_t bytes, void** ptr, tcx_hip_pool_t** owner);
/* Returns a block from tcx_hip_allocate: to its pool's cache when that pool
 * is still active and has room, else hipFree. Never fails the caller. */
void tcx_hip_release(void* ptr, size_t bytes, tcx_hip_pool_t* owner);
/* tcx_hip_release that never caches the block: storage that was exposed to
 * another framework (DLPack export, copies included) may still be read by
 * work on streams this library cannot see, so it goes straight back to
 * hipFree, which waits for the device (the reference's exported-buffer rule,
 * bindings/dlpack.cpp:204-206 and cuda_buffer.h:35). */
void tcx_hip_release_uncached(void* ptr, size_t bytes, tcx_hip_pool_t* owner);

/* Checks memory handed over by another framework before a tensor borrows it
 * (replaces the checks of CudaBuffer::borrow, cuda_backend.cpp:106-144):
 * [ptr, ptr + bytes) must be device memory of device 0 inside one allocation.
 * Then it waits for all work on the device, so the producer's writes on any
 * of its streams are complete before the borrowed storage is read. bytes == 0
 * only waits. */
int tcx_hip_borrow_check(const void* ptr, size_t bytes);

/* Copies on `stream`, synchronised before return (cuda::from_cpu/to_cpu,
 * cuda_backend.cpp:215-264). */
int tcx_hip_memcpy_h2d(void* dst, const void* src, size_t bytes, tcx_stream_t stream);
int tcx_hip_memcpy_d2h(void* dst, const void* src, size_t bytes, tcx_stream_t stream);
int tcx_hip_memcpy_d2d(void* dst, const void* src, size_t bytes, tcx_stream_t stream);

/* ---------------------------------------------------------- bounded pool */

/* Injectable allocator seam (reference cuda_memory_pool.h:20-27) so pool
 * logic is testable without a device. Each returns a TCX_* code;
 * allocate returns TCX_UNAVAILABLE+100 (TCX_POOL_OOM) for out-of-memory. */
#define TCX_POOL_OOM 102
typedef struct {
  int (*allocate)(void** ptr, size_t bytes);
  int (*free)(void* ptr);
  int (*clear_error)(void);
} tcx_hip_pool_runtime_t;

typedef struct {
  size_t max_cached_bytes, max_cached_blocks, cached_bytes, cached_blocks;
  size_t in_use_bytes, peak_in_use_bytes, peak_cached_bytes;
  uint64_t hits, misses, allocation_calls, free_calls, allocation_failures, oom_retries,
      uncached_returns, readiness_failures, free_failures, failed_free_bytes;
  int active;
} tcx_hip_pool_stats_t;

/* Bounded exact-size block cache with the semantics of the reference's
 * MemoryPool (cuda_memory_pool.cpp:21-163): thread-scoped, single-use,
 * not nestable; on allocation OOM with blocks cached it drains the cache and
 * retries once. `runtime` may be NULL for hipMalloc/hipFree. */
int tcx_hip_pool_create(size_t max_cached_bytes, size_t max_cached_blocks,
                        const tcx_hip_pool_runtime_t* runtime, tcx_hip_pool_t** pool);
int tcx_hip_pool_enter(tcx_hip_pool_t* pool);
int tcx_hip_pool_exit(tcx_hip_pool_t* pool);
int tcx_hip_pool_trim(tcx_hip_pool_t* pool);
int tcx_hip_pool_stats(const tcx_hip_pool_t* pool, tcx_hip_pool_stats_t* stats);
/* Drops the caller's reference; cached blocks are freed when the last
 * outstanding buffer from the pool has been released. */
void tcx_hip_pool_destroy(tcx_hip_pool_t* pool);

/* ------------------------------------------------------------------- events */

/* Device timing (the reference's DeviceTimer, cuda_profiling.h:22-77). */
int tcx_hip_event_create(void** event);
int tcx_hip_event_record(void* event, tcx_stream_t stream);
int tcx_hip_event_synchronize(void* event);
int tcx_hip_event_elapsed_ms(void* start, void* stop, float* ms);
int tcx_hip_event_destroy(void* event);

/* ------------------------------------------------------------------ kernels */

#define TCX_HIP_MAX_BATCH_RANK 8

#define TCX_ACT_NONE 0
#define TCX_ACT_SILU 1
#define TCX_ACT_GELU 2

typedef struct {
  int64_t m, n, k;
  int64_t batch_count;                          /* product of batch_shape (1 if rank 0) */
  int32_t batch_rank;                           /* <= TCX_HIP_MAX_BATCH_RANK */
  int32_t rhs_transposed;                       /* 1: rhs is [n, k] row-major */
  int64_t batch_shape[TCX_HIP_MAX_BATCH_RANK];
  int64_t lhs_batch_strides[TCX_HIP_MAX_BATCH_RANK]; /* in elements */
  int64_t rhs_batch_strides[TCX_HIP_MAX_BATCH_RANK];
  const float* bias;                            /* optional [n], added per column */
  int32_t activation;                           /* TCX_ACT_*, applied after bias */
} tcx_hip_gemm_desc_t;

/* out[b] = act(lhs[b] @ rhs[b] (+ bias)), fp32 on v_mfma_f32_16x16x4_f32,
 * out contiguous [batch..., m, n]. Replaces launch_matmul
 * (reference backends/cuda/cuda_kernels.h:11-45; kernels/primitives.cu:251-333)
 * and, with rhs_transposed + bias, the kLinear composite
 * (core/inference.cpp:89-102) without its transpose copy. */
int tcx_hip_gemm_f32(const float* lhs, const float* rhs, float* out,
                     const tcx_hip_gemm_desc_t* desc, tcx_stream_t stream);

/* Workspace bytes that tcx_hip_gemm_f32_ws can use for desc: > 0 when the
 * shape has few output tiles and a long K, which then runs with K split over
 * several blocks whose partial sums land in the workspace, or when an
 * unbatched product's K or N is not a multiple of 4 (zero-padded copies of
 * A, B and the output, so that the 16-byte kernels run); 0 otherwise. */
size_t tcx_hip_gemm_workspace_bytes(const tcx_hip_gemm_desc_t* desc);
/* tcx_hip_gemm_f32 with that workspace (16-byte aligned). With NULL or fewer
 * bytes than the query it runs unsplit. Same results to the matmul bar (the
 * split partial sums are added in split order, then bias and activation);
 * the workspace must stay allocated until the stream has run the call. Same
 * reference interfaces as tcx_hip_gemm_f32. */
int tcx_hip_gemm_f32_ws(const float* lhs, const float* rhs, float* out,
                        const tcx_hip_gemm_desc_t* desc, void* workspace,
                        size_t workspace_bytes, tcx_stream_t stream);

#define TCX_REDUCE_SUM 0
#define TCX_REDUCE_MAX 1
#define TCX_REDUCE_MEAN 2
#define TCX_REDUCE_MIN 3
#define TCX_REDUCE_ARGMAX 4

/* Reduction of x viewed as [outer, reduce, inner] over the middle axis into
 * out [outer, inner]: the single-axis reduce of cpu_backend.cpp:1154-1249
 * and min/argmax of cpu_math.cpp:27-76 (argmax writes int32 indices), and any
 * multi-axis selection whose reduced axes are adjacent. dtype TCX_FLOAT32
 * (sum, max, mean, min, argmax) or TCX_INT32 (sum wrapping mod 2^32, max,
 * min, argmax). workspace may be NULL when the query returns 0. */
size_t tcx_hip_reduce_workspace_bytes(int op, int dtype, int64_t outer, int64_t reduce,
                                      int64_t inner);
int tcx_hip_reduce(int op, int dtype, const void* x, void* out, int64_t outer, int64_t reduce,
                   int64_t inner, void* workspace, size_t workspace_bytes, tcx_stream_t stream);

/* Metadata capacity of tcx_hip_reduce_axes and tcx_hip_binary. Callers fold
 * the shape first (size-1 axes dropped, neighbouring axes that every operand
 * walks alike merged), which leaves every axis with extent >= 2, so a folded
 * rank above 40 would need more than 2^40 elements: any tensor that fits in
 * device memory folds within it. */
#define TCX_HIP_MAX_FOLDED_RANK 40

/* tcx_hip_reduce without a workspace, for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); it has no counterpart in the reference. It runs the kernels of
 * tcx_hip_reduce with the partials of split plans (few long rows, e.g. a
 * full-tensor sum; few columns over many rows) in a static per-device
 * scratch of 4 MiB, held until the process ends, so its results are
 * bit-identical to
 * tcx_hip_reduce's. Plans are accepted when tcx_hip_reduce_workspace_bytes is
 * at most TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE (else TCX_INVALID_ARGUMENT),
 * which holds for every float32 or int32 input that fits in 288 GB. All calls
 * on one GPU share the scratch: calls that overlap in time on one GPU (other
 * streams, other threads) race and must be serialised by the caller. It
 * never allocates. */
#define TCX_HIP_REDUCE_NOALLOC_MAX_WORKSPACE 4194304
int tcx_hip_reduce_noalloc(int op, int dtype, const void* x, void* out, int64_t outer, int64_t reduce,
                           int64_t inner, tcx_stream_t stream);

/* General reduction over any axis selection, with the reference's
 * make_reduction_plan metadata (core/shape.cpp:140-173): `meta` holds
 * extent/stride pairs for all `rank` (<= TCX_HIP_MAX_FOLDED_RANK) axes, kept
 * axes first then reduced axes, `outer_rank` of them kept; one output per
 * group in the reference's exact element order (cpu_backend.cpp:1102-1153;
 * cpu_math.cpp:48-54). */
int tcx_hip_reduce_axes(int op, int dtype, const void* x, void* out, const int64_t* meta,
                        int32_t outer_rank, int32_t rank, int64_t groups,
                        int64_t reduction_size, tcx_stream_t stream);

/* Row softmax / RMSNorm / LayerNorm of x viewed as [outer, reduce, inner] over
 * the middle axis (cpu_backend.cpp:125-240). gamma/beta are optional [reduce]
 * affine parameters applied as two separately rounded steps, which is the
 * kAffine*Norm composite of core/inference.cpp:103-122 fused into one pass. */
int tcx_hip_softmax_f32(const float* x, float* out, int64_t outer, int64_t reduce,
                        int64_t inner, tcx_stream_t stream);
int tcx_hip_rmsnorm_f32(const float* x, const float* gamma, float* out, int64_t outer,
                        int64_t reduce, int64_t inner, float eps, tcx_stream_t stream);
int tcx_hip_layernorm_f32(const float* x, const float* gamma, const float* beta, float* out,
                          int64_t outer, int64_t reduce, int64_t inner, float eps,
                          tcx_stream_t stream);

/* The same row ops with a workspace (the reference has one entry per op,
 * cpu_backend.cpp:125-240; these add the workspace argument). Over a middle
 * axis (inner > 1) whose column tiles are too few to fill the GPU, the rows
 * of each column are split over blocks: per-split statistics go to the
 * workspace, then a fold and a write pass (three launches). Without a
 * workspace (the entry points above) a strided op runs unsplit in one launch.
 * tcx_hip_rownorm_workspace_bytes gives the size (0: none needed; at most
 * 16 MiB); a smaller workspace is TCX_INVALID_ARGUMENT. */
size_t tcx_hip_rownorm_workspace_bytes(int64_t outer, int64_t reduce, int64_t inner);
int tcx_hip_softmax_f32_ws(const float* x, float* out, int64_t outer, int64_t reduce, int64_t inner,
                           void* workspace, size_t workspace_bytes, tcx_stream_t stream);
int tcx_hip_rmsnorm_f32_ws(const float* x, const float* gamma, float* out, int64_t outer,
                           int64_t reduce, int64_t inner, float eps, void* workspace,
                           size_t workspace_bytes, tcx_stream_t stream);
int tcx_hip_layernorm_f32_ws(const float* x, const float* gamma, const float* beta, float* out,
                             int64_t outer, int64_t reduce, int64_t inner, float eps,
                             void* workspace, size_t workspace_bytes, tcx_stream_t stream);

/* out[r, c] = act(x[r, c] + bias[c]) (bias optional): fused bias+activation,
 * the kAdd-broadcast of kLinear followed by kSilu/kGelu (cpu_backend.cpp:
 * 1004-1006, 1014-1097) in one pass. */
int tcx_hip_bias_act_f32(const float* x, const float* bias, float* out, int64_t rows,
                         int64_t cols, int activation, tcx_stream_t stream);

#define TCX_UNARY_EXP 0
#define TCX_UNARY_GELU 1
#define TCX_UNARY_SILU 2
/* Elementwise exp/gelu/silu (cpu_backend.cpp:1000-1010). */
int tcx_hip_unary_f32(int op, const float* x, float* out, int64_t n, tcx_stream_t stream);

#define TCX_BINARY_ADD 0
#define TCX_BINARY_SUBTRACT 1
#define TCX_BINARY_MULTIPLY 2
#define TCX_BINARY_DIVIDE 3
#define TCX_HIP_MAX_RANK 8
/* Broadcast arithmetic over a make_broadcast_plan (core/shape.cpp:202-229) of
 * `rank` <= TCX_HIP_MAX_FOLDED_RANK axes: float32, or int32 wrapping (no
 * divide) as in cpu_backend.cpp:1014-1097. */
int tcx_hip_binary(int op, int dtype, const void* lhs, const void* rhs, void* out, int32_t rank,
                   const int64_t* out_shape, const int64_t* lhs_strides,
                   const int64_t* rhs_strides, tcx_stream_t stream);

/* kFill (cpu_backend.cpp fill): float32, int32 or bool (value != 0) into n elements. */
int tcx_hip_fill(int dtype, void* out, int64_t n, double value, tcx_stream_t stream);

/* ---- data movement and conversion (replaces the CUDA executor paths of
 * reference backends/cuda/kernels/elementwise.cu; semantics of
 * backends/cpu/cpu_backend.cpp:801-930) ---- */

/* kTranspose / kSlice (make_transpose_plan, make_slice_plan, shape.cpp:87-200):
 * out (contiguous over out_shape) [i] = in[offset + sum_a idx_a(i) * in_strides[a]],
 * bit for bit, for 1- or 4-byte elements. */
int tcx_hip_gather_strided(int elem_bytes, const void* in, void* out, int32_t rank, const int64_t* out_shape,
                           const int64_t* in_strides, int64_t offset, tcx_stream_t stream);
/* One kConcat input (cpu_backend.cpp:317-339): a contiguous [outer, block]
 * input copied into out at out[o * out_block + dst_offset + j]. */
int tcx_hip_copy_blocks(int elem_bytes, const void* in, void* out, int64_t outer, int64_t block, int64_t out_block,
                        int64_t dst_offset, tcx_stream_t stream);
/* kCast (cpu_backend.cpp:834-876) between TCX_FLOAT32 / TCX_INT32 / TCX_BOOL:
 * to/from bool tests value != 0; float32 -> int32 truncates toward zero after
 * every value was checked finite and inside [-2^31, 2^31) (else
 * TCX_INVALID_ARGUMENT; `flag` is one device int32 of scratch and the stream
 * is synchronised for that check); int32 -> float32 rounds to nearest. */
int tcx_hip_cast(int from_dtype, int to_dtype, const void* in, void* out, int64_t n, int32_t* flag,
                 tcx_stream_t stream);

#define TCX_SCALAR_NEGATE 0
#define TCX_SCALAR_ADD 1
#define TCX_SCALAR_SUBTRACT 2
#define TCX_SCALAR_MULTIPLY 3
#define TCX_SCALAR_DIVIDE 4
/* kNegate and k{Add,Subtract,Multiply,Divide}Scalar (cpu_backend.cpp:878-930):
 * float32 with the scalar rounded to float32 once, int32 wrapping in uint32
 * (no division; the scalar must be an int32 integer); scalar_left puts the
 * scalar on the left. */
int tcx_hip_scalar_op(int op, int dtype, const void* in, void* out, int64_t n, double scalar, int scalar_left,
                      tcx_stream_t stream);

/* ---- predicates (replace reference backends/cuda/kernels/predicate.cu;
 * semantics of backends/cpu/cpu_predicate.cpp) ---- */
#define TCX_PRED_EQUAL 0
#define TCX_PRED_NOT_EQUAL 1
#define TCX_PRED_LESS 2
#define TCX_PRED_LESS_EQUAL 3
#define TCX_PRED_GREATER 4
#define TCX_PRED_GREATER_EQUAL 5
#define TCX_PRED_LOGICAL_AND 6
#define TCX_PRED_LOGICAL_OR 7
#define TCX_PRED_LOGICAL_XOR 8
#define TCX_PRED_LOGICAL_NOT 9
#define TCX_PRED_WHERE 10
#define TCX_PRED_FLAG_INT32 1 /* 4-byte comparisons are int32 (else float32) */
typedef struct {
  int64_t shape[TCX_HIP_MAX_RANK];      /* broadcast output shape */
  int64_t strides[3][TCX_HIP_MAX_RANK]; /* broadcast strides of inputs a, b, c */
  int32_t rank;
  int32_t flags;                        /* TCX_PRED_FLAG_* */
} tcx_hip_broadcast3_t;
/* make_predicate_plan (core/predicate.cpp:23-44), cpu_predicate.cpp:22-50:
 * comparisons of a and b (elem_bytes 4: float32 or int32 per flags; 1: bool)
 * and logical ops of bool a (, b) into bool out; where(a: bool, b, c) copies
 * the chosen elem_bytes-wide element bit for bit. */
int tcx_hip_predicate(int op, int elem_bytes, const void* a, const void* b, const void* c, void* out,
                      const tcx_hip_broadcast3_t* plan, tcx_stream_t stream);
/* kAny (all == 0) / kAll over make_reduction_plan metadata (core/shape.cpp:
 * 140-173; cpu_predicate.cpp:52-70): (extent, stride) pairs of `rank` axes,
 * kept axes first; false / true for an empty selection. */
int tcx_hip_bool_reduce(int all, const uint8_t* x, uint8_t* out, const int64_t* meta, int32_t rank, int64_t groups,
                        int64_t reduce, tcx_stream_t stream);
/* kMaskedSelect (cpu_predicate.cpp:72-96) in two launches around one host
 * step: tcx_hip_mask_count writes the true entries of each of the
 * tcx_hip_mask_chunks(n) chunks of the n-entry bool mask; the caller turns
 * them into exclusive offsets and the total, then tcx_hip_masked_select writes
 * the selected entry indices (`index`, total int64 of scratch) and copies the
 * `block`-element rows of `in` they select to `out`, in index order. */
int64_t tcx_hip_mask_chunks(int64_t n);
int tcx_hip_mask_count(const uint8_t* mask, int64_t n, int64_t* chunk_counts, tcx_stream_t stream);
int tcx_hip_masked_select(int elem_bytes, const void* in, const uint8_t* mask, int64_t n, int64_t block,
                          const int64_t* chunk_offsets, int64_t total, int64_t* index, void* out,
                          tcx_stream_t stream);

/* ---- math extension (replaces the CUDA math launches of reference
 * backends/cuda/kernels/math.cu; semantics of backends/cpu/cpu_math.cpp) ---- */
#define TCX_MATH_LOG 0
#define TCX_MATH_SQRT 1
#define TCX_MATH_ABS 2
/* kLog / kSqrt (float32) and kAbs (float32 sign clear; int32 negation in uint32,
 * so INT32_MIN stays) over n contiguous elements (cpu_math.cpp:40-44). */
int tcx_hip_math_unary(int op, int dtype, const void* x, void* out, int64_t n, tcx_stream_t stream);

/* kClip over a three-way broadcast plan (math.cpp:32-38): out_shape of `rank`
 * axes and the broadcast strides of x, lo and hi (cpu_math.cpp:45-50). */
int tcx_hip_clip(int dtype, const void* x, const void* lo, const void* hi, void* out, int32_t rank,
                 const int64_t* out_shape, const int64_t* x_strides, const int64_t* lo_strides,
                 const int64_t* hi_strides, tcx_stream_t stream);

/* kTopK along the middle extent of (outer, reduce, inner) (math.cpp:56-66,
 * cpu_math.cpp:57-67): values (x's dtype) and int32 indices of shape
 * (outer, k, inner). NaN first when largest (last otherwise), ties by lower
 * index; sorted == 0 lists the chosen k in index order. */
int tcx_hip_topk(int dtype, const void* x, void* values, int32_t* indices, int64_t outer, int64_t reduce,
                 int64_t inner, int64_t k, int largest, int sorted, tcx_stream_t stream);

/* ---- inference primitives (replace reference backends/cuda/kernels/
 * inference.cu; semantics of backends/cpu/cpu_inference.cpp) ---- */

/* kEmbedding (cpu_inference.cpp:12-21): out[i, :] = weight[indices[i], :] for
 * `count` indices into a (vocabulary, width) table, copied bit for bit. Every
 * index is checked on the device, also when width is 0; an index outside
 * [0, vocabulary) returns TCX_INVALID_ARGUMENT (out is then unspecified).
 * `flag` is one caller-provided device int32 of scratch. Synchronizes
 * `stream` to read the check back. */
int tcx_hip_embedding_f32(const int32_t* indices, const float* weight, float* out, int64_t count,
                          int64_t vocabulary, int64_t width, int32_t* flag, tcx_stream_t stream);

#define TCX_MASK_NONE 0
#define TCX_MASK_BOOL 1     /* 1-byte bool, false masks the score out */
#define TCX_MASK_ADDITIVE 2 /* float32 added to the scaled score */
typedef struct {
  int64_t shape[TCX_HIP_MAX_RANK];         /* attention shape (..., queries, keys) */
  int64_t score_strides[TCX_HIP_MAX_RANK]; /* broadcast strides of the scores */
  int64_t mask_strides[TCX_HIP_MAX_RANK];  /* broadcast strides of the mask */
  int32_t rank;                            /* 2..TCX_HIP_MAX_RANK */
  int32_t mask_kind;                       /* TCX_MASK_* */
  int32_t causal;                          /* key > query % queries masked out */
  float scale;                             /* checked float32 scale */
} tcx_hip_attention_softmax_desc_t;
/* kAttentionSoftmax (make_attention_softmax_plan, inference.cpp:59-84;
 * cpu_inference.cpp:22-47): per row, scores * scale + mask bias with causal /
 * bool / -inf masking, NaN-first maximum, a row with maximum -inf is zeros,
 * else exp(s - max) / sum. `out` is contiguous in `shape`. */
int tcx_hip_attention_softmax_f32(const float* scores, const void* mask, float* out,
                                  const tcx_hip_attention_softmax_desc_t* desc, tcx_stream_t stream);

/* 1 when tcx_hip_flash_attention_f32 handles these feature sizes
 * (features == value_features, one of 32, 64, 128), else 0. */
int tcx_hip_flash_attention_supported(int64_t features, int64_t value_features);
/* Fused kAttention without a mask (core/inference.cpp:123-161 with
 * cpu_inference.cpp:22-47): out[b] = softmax(scale * q[b] k[b]^T, causal) v[b]
 * for `batch` contiguous matrices q [rows, features], k and v [cols, features],
 * out [rows, features], 16-byte aligned, never materialising the scores.
 * Causal masks key j > query i. Replaces the three launches of the reference's
 * attention composite (transpose, matmul, softmax, matmul). */
int tcx_hip_flash_attention_f32(const float* q, const float* k, const float* v, float* out, int64_t batch,
                                int64_t rows, int64_t cols, int64_t features, float scale, int causal,
                                tcx_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* TENSORCX_HIP_H_ */
