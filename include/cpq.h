/*
 * cpq.h -- C ABI of the MI355X (gfx950) affine group-quantized matmul library
 * (libcpq.so).  Drop-in boundary for the reference's quantized-matmul path:
 * the kernels crate's dispatch/buffer layer and op API
 * (crates/cider-press-kernels/src/{device,buffer,commands,error}.rs and
 * kernels/{qmv,qmm,dequantize}.rs) and the runtime's QuantizedMatMul node
 * (crates/cider-press-runtime/src/{quantization,quantized,tensor,eval}.rs).
 *
 * Conventions
 *  - Plain pointers and element counts; no framework types.  16-bit floats
 *    are passed as `const void*` and interpreted per `cpq_dtype`.
 *  - Ops ENCODE ONLY: they validate, enqueue on the session's HIP stream and
 *    return.  Nothing synchronises until cpq_commands_wait / commit_and_wait
 *    (reference: kernels/mod.rs:1-9 "functions never commit").
 *  - Every shape/divisibility violation returns CPQ_ERR_INVALID_ARGUMENT
 *    before any launch; an unsupported (dtype, group_size, bits) returns
 *    CPQ_ERR_KERNEL_NOT_FOUND; a failed stream surfaces at wait as
 *    CPQ_ERR_COMMAND_BUFFER_FAILED.  The message of the last failure on the
 *    calling thread is cpq_last_error_message().
 *  - Caller owns all device buffers.  Quantized weights are never written.
 *  - Thread safety: one thread drives a given cpq_commands at a time; the
 *    library itself holds no mutable global state besides per-thread error
 *    text and the per-device kernel property cache.
 */
#ifndef CPQ_H
#define CPQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Error classes; mirror cider_press_kernels::Error (error.rs:15-70). */
typedef enum cpq_status {
  CPQ_OK = 0,
  CPQ_ERR_NO_DEVICE = 1,             /* Error::NoDevice            error.rs:21-23 */
  CPQ_ERR_KERNEL_NOT_FOUND = 2,      /* Error::KernelNotFound      error.rs:30-34 */
  CPQ_ERR_BUFFER_ALLOCATION = 3,     /* Error::BufferAllocation    error.rs:40-42 */
  CPQ_ERR_BUFFER_TOO_LARGE = 4,      /* Error::BufferTooLarge      error.rs:44-48 */
  CPQ_ERR_INVALID_ARGUMENT = 5,      /* Error::InvalidArgument     error.rs:56-61 */
  CPQ_ERR_COMMAND_BUFFER_FAILED = 6, /* Error::CommandBufferFailed error.rs:63-69 */
  CPQ_ERR_HIP_API = 7,               /* Error::AppleApi analogue   error.rs:50-54 */
  /* Loader errors of the models crate (cider-press-models/src/error.rs:9-60). */
  CPQ_ERR_MISSING_KEY = 8,           /* Error::MissingKey          error.rs:12-16 */
  CPQ_ERR_UNSUPPORTED_DTYPE = 9,     /* Error::UnsupportedDtype    error.rs:18-24 */
  CPQ_ERR_SHAPE_MISMATCH = 10,       /* Error::ShapeMismatch       error.rs:26-34 */
  CPQ_ERR_SAFETENSORS = 11,          /* Error::Safetensors         error.rs:36-38 */
  CPQ_ERR_JSON = 12                  /* Error::Json                error.rs:40-41 */
} cpq_status;

/* Activation / scale / bias / output element type (T). */
typedef enum cpq_dtype {
  CPQ_DTYPE_F32 = 0, /* accepted by validators; no f32 kernels are built */
  CPQ_DTYPE_F16 = 1,
  CPQ_DTYPE_BF16 = 2,
  CPQ_DTYPE_U32 = 3  /* index tensors of the runtime graph (token ids); never a T */
} cpq_dtype;

typedef struct cpq_device cpq_device;
typedef struct cpq_commands cpq_commands;
typedef struct cpq_event cpq_event;
typedef struct cpq_qweight cpq_qweight;
typedef struct cpq_tensor cpq_tensor;

/* ------------------------------------------------------------------ */
/* Errors and version                                                   */
/* ------------------------------------------------------------------ */

/* Text of the last non-OK status returned on this thread ("" if none). */
const char* cpq_last_error_message(void);
const char* cpq_version(void);

/* ------------------------------------------------------------------ */
/* Device and buffers (kernels/src/device.rs, buffer.rs)                */
/* ------------------------------------------------------------------ */

/* Device::system_default (device.rs:77): HIP device 0.  CPQ_ERR_NO_DEVICE if absent. */
cpq_status cpq_device_system_default(cpq_device** out);
void cpq_device_release(cpq_device* dev);
/* Marketing name, compute-unit count and peak clock (kHz) of the device. */
cpq_status cpq_device_info(cpq_device* dev, char* name, size_t name_cap, int* cu_count,
                           int* clock_khz);

/* Device::alloc_buffer (device.rs:167-228): allocation rounded up to 512 B,
 * the slack past byte_len zeroed (the K-padding contract of qmv.rs:95-124).
 * *out_alloc_len receives the rounded length (Buffer::metal_alloc_len). */
cpq_status cpq_alloc_buffer(cpq_device* dev, size_t byte_len, void** out_ptr,
                            size_t* out_alloc_len);
/* Device::upload (device.rs:233): alloc_buffer + synchronous host->device copy. */
cpq_status cpq_upload(cpq_device* dev, const void* host, size_t byte_len, void** out_ptr,
                      size_t* out_alloc_len);
cpq_status cpq_free_buffer(cpq_device* dev, void* ptr);
/* Synchronous copies (Buffer::as_slice / as_mut_slice after a wait, buffer.rs:176-199). */
cpq_status cpq_read_buffer(cpq_device* dev, const void* dev_ptr, void* host, size_t byte_len);
cpq_status cpq_write_buffer(cpq_device* dev, void* dev_ptr, const void* host, size_t byte_len);

/* ------------------------------------------------------------------ */
/* Command sessions (kernels/src/commands.rs): one in-order HIP stream   */
/* ------------------------------------------------------------------ */

/* Device::commands (device.rs:319): a new session on its own HIP stream. */
cpq_status cpq_commands_create(cpq_device* dev, cpq_commands** out);
/* Wrap a caller-owned hipStream_t (e.g. a framework's current stream). */
cpq_status cpq_commands_wrap_stream(cpq_device* dev, void* hip_stream, cpq_commands** out);
void* cpq_commands_stream(cpq_commands* cmds);
/* Commands::commit (commands.rs:349-359): work is already submitted on HIP; a no-op flush. */
cpq_status cpq_commands_commit(cpq_commands* cmds);
/* CommandsInFlight::wait (commands.rs:416-419): hipStreamSynchronize; a stream
 * failure maps to CPQ_ERR_COMMAND_BUFFER_FAILED (commands.rs:381-400). */
cpq_status cpq_commands_wait(cpq_commands* cmds);
cpq_status cpq_commands_commit_and_wait(cpq_commands* cmds);
void cpq_commands_release(cpq_commands* cmds);

/* HIP graph capture of a session's stream: everything encoded between begin
 * and end is recorded (not run) and replayed by cpq_graph_launch.  No op of
 * this library records a memset, so captured graphs replay identically.  No
 * counterpart in the reference (Metal command buffers are re-encoded per
 * call); used for decode loops and for launch-overhead-free timing. */
typedef struct cpq_graph cpq_graph;
cpq_status cpq_commands_begin_capture(cpq_commands* cmds);
cpq_status cpq_commands_end_capture(cpq_commands* cmds, cpq_graph** out);
cpq_status cpq_graph_launch(cpq_graph* graph, cpq_commands* cmds);
void cpq_graph_release(cpq_graph* graph);

/* Encoder hazard hooks of the reference's runtime (commands.rs:139-153
 * record_output / record_input / record_unresolved_input, commands.rs:290-296
 * elide_next_barrier), called by its graph evaluator around every op
 * (eval.rs:280-292, 450-462).  They feed Metal's cross-encoder fences and
 * per-dispatch buffer barriers.  A session here is one in-order HIP stream,
 * so every launch already starts after the previous one has finished and
 * there is no fence or barrier to add or elide: the hooks check the session
 * and return CPQ_OK, and ops behave exactly as without them.  Eliding a
 * barrier is only ever an allowed overlap in the reference, never required.
 * (dispatch_threads / dispatch_threadgroups, commands.rs:298-330, have no
 * counterpart: every op launches its own grid.) */
cpq_status cpq_commands_record_input(cpq_commands* cmds, uint64_t key);
cpq_status cpq_commands_record_output(cpq_commands* cmds, uint64_t key);
cpq_status cpq_commands_record_unresolved_input(cpq_commands* cmds);
cpq_status cpq_commands_elide_next_barrier(cpq_commands* cmds);

/* Per-op GPU timing of a session (GpuSampler, gpu_sampler.rs:44-162, and the
 * profiled-session calls of commands.rs:155-181, 361-374, 465-470). */

/* One timed op: its label and its GPU execution window in ticks
 * (GpuSegment, gpu_sampler.rs:22-42).  Ticks are nanoseconds on the GPU's
 * timeline, counted from the start of the batch's first op. */
typedef struct cpq_gpu_segment {
  const char* label; /* valid until the next resolve or the session's release */
  uint64_t start_tick;
  uint64_t end_tick;
} cpq_gpu_segment;

/* Device::supports_stage_boundary_sampling (device.rs:314-322): 1.  A timing
 * event can be recorded between any two launches of an in-order stream. */
int cpq_device_supports_stage_boundary_sampling(cpq_device* dev);
/* Device::gpu_timestamp_period_ns (device.rs:324-368): nanoseconds per tick
 * of cpq_gpu_segment, 1.0 here. */
cpq_status cpq_device_gpu_timestamp_period_ns(cpq_device* dev, double* out_ns_per_tick);
/* Device::commands_profiled / Commands::new_profiled (commands.rs:155-161,
 * 465-470): a session that can time up to op_capacity ops per batch (two
 * timing events each, created here).  CPQ_ERR_HIP_API if op_capacity * 2
 * overflows or the events cannot be created. */
cpq_status cpq_commands_create_profiled(cpq_device* dev, size_t op_capacity, cpq_commands** out);
/* Commands::begin_profiled_op (commands.rs:163-181): ends the open op's
 * window (if any) and opens one for `label` (copied) covering everything
 * encoded until the next begin_profiled_op or commit_wait_resolve.  No-op on
 * an ordinary session.  Past op_capacity ops it stops timing further ops
 * instead of failing (the resolved batch has fewer segments).  The GPU runs
 * work as it is encoded, so an op's window also holds any time the GPU sat
 * idle waiting for the host to encode it.  CPQ_ERR_INVALID_ARGUMENT while
 * the stream is being captured into a graph. */
cpq_status cpq_commands_begin_profiled_op(cpq_commands* cmds, const char* label);
/* Ops recorded in the current batch, and the timestamp capacity (2 per op:
 * GpuSampler::recorded_segments().len(), sample_capacity()). */
cpq_status cpq_commands_profiled_info(cpq_commands* cmds, size_t* recorded_ops, size_t* sample_capacity);
/* Commands::commit_wait_resolve (commands.rs:361-374) with
 * GpuSampler::resolve (gpu_sampler.rs:121-162): ends the open op's window,
 * waits for the session exactly as cpq_commands_wait (same statuses), then
 * writes one segment per recorded op, in encode order, to out[0..*n_out)
 * and starts a new batch.  cap must hold the recorded ops
 * (CPQ_ERR_INVALID_ARGUMENT before waiting otherwise).  On an ordinary
 * session: waits and returns 0 segments. */
cpq_status cpq_commands_commit_wait_resolve(cpq_commands* cmds, cpq_gpu_segment* out, size_t cap,
                                            size_t* n_out);

/* Maps the HIP status of a finished stream to the status cpq_commands_wait
 * returns (commands.rs:378-400 completion_result): CPQ_OK for hipSuccess,
 * else CPQ_ERR_COMMAND_BUFFER_FAILED with the HIP error's name and text as
 * the message.  Exported so the mapping can be checked without a failing
 * GPU. */
cpq_status cpq_completion_result(int hip_error);

/* GPU timing on a session's stream between two recorded events. */
cpq_status cpq_event_create(cpq_event** out);
cpq_status cpq_event_record(cpq_event* ev, cpq_commands* cmds);
cpq_status cpq_event_elapsed_ms(cpq_event* start, cpq_event* end, float* out_ms);
void cpq_event_release(cpq_event* ev);

/* Streaming read of up to 4 device regions (16-byte aligned, lengths
 * multiples of 16) in one launch of n_workgroups x 256 threads; `sink` (one
 * device u32) is written only in the practically impossible case that the
 * XOR of everything read equals a fixed 128-bit constant.  Measurement
 * support: the HBM ceiling of one launch over a given byte count, timed
 * beside the kernels it bounds.  No reference counterpart (its benches
 * compare against the spec bandwidth, tests/qmv_dispatch_bench.rs:37-79). */
cpq_status cpq_stream_read(cpq_commands* cmds, const void* const* regions, const size_t* bytes, int n_regions,
                           uint32_t* sink, int n_workgroups);

/* The same read in one of cpq_stream_read_variant_count() designs (variant 0
 * is cpq_stream_read's): workgroups of 256, 512 or 1024 threads, 4, 8 or 16
 * loads in flight per lane, plain or non-temporal loads, global or buffer
 * addressing.  The benchmark takes the fastest as the ceiling.  At most
 * 4 GiB per workgroup. */
cpq_status cpq_stream_read_variant(cpq_commands* cmds, const void* const* regions, const size_t* bytes,
                                   int n_regions, uint32_t* sink, int n_workgroups, int variant);
int cpq_stream_read_variant_count(void);

/* ------------------------------------------------------------------ */
/* Quantization descriptor (runtime/src/quantization.rs:43-153)          */
/* ------------------------------------------------------------------ */

/* Quantization::validate (quantization.rs:86-106): bits in {2,3,4,5,6,8},
 * group_size a positive power of two, group_size*bits % 32 == 0. */
cpq_status cpq_quantization_validate(uint32_t bits, uint32_t group_size);
/* Quantization::packed_word_count (quantization.rs:121-141). */
cpq_status cpq_packed_word_count(uint32_t bits, uint32_t group_size, size_t scalar_count,
                                 size_t* out);
/* Quantization::group_count (quantization.rs:145-153). */
cpq_status cpq_group_count(uint32_t bits, uint32_t group_size, size_t scalar_count,
                           size_t* out);
/* KernelLibrary::pipeline lookup (library.rs:264-286): 1 if a kernel for
 * (dtype, group_size, bits) is built, else 0. */
int cpq_kernel_available(cpq_dtype dtype, uint32_t group_size, uint32_t bits);

/* ------------------------------------------------------------------ */
/* Ops (kernels/src/kernels/{qmv,qmm,dequantize}.rs)                     */
/* ------------------------------------------------------------------ */

/* affine_qmv_bf16 (qmv.rs:77-205), any T: y[N] = x . dequant(w_q)^T for one
 * activation row.  in_vec_size is the PHYSICAL K of the weight; x may be a
 * K-padded activation whose allocation (x_alloc_bytes) covers K*sizeof(T)
 * with a zeroed tail.  N = y_len.  w_q_len = N*K*bits/32,
 * scales_len = biases_len = N*K/group_size. */
cpq_status cpq_affine_qmv(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                          size_t w_q_len, const void* scales, size_t scales_len,
                          const void* biases, size_t biases_len, const void* x,
                          size_t x_alloc_bytes, void* y, size_t y_len, size_t in_vec_size,
                          uint32_t group_size, uint32_t bits);

/* affine_qmm_t_bf16 (qmm.rs:66-220), any T: Y[M,N] = X[M,K] . dequant(W[N,K])^T.
 * N % 32 == 0 is required as in the reference's aligned variant (qmm.rs:101-106).
 * The kernel is chosen by M as for cpq_quantized_matmul's M > 1 case
 * (small-M kernels up to 64 rows, 32 past N = 8192; else the prefill plan). */
cpq_status cpq_affine_qmm_t(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                            size_t w_q_len, const void* scales, size_t scales_len,
                            const void* biases, size_t biases_len, const void* x, size_t x_len,
                            void* y, size_t y_len, size_t m, size_t n, size_t k,
                            uint32_t group_size, uint32_t bits);

/* affine_qmm_t for callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, hosts that forbid allocation after
 * start-up).  No counterpart in the reference.  Same validation and numerics
 * as cpq_affine_qmm_t, enqueued on the caller's hipStream_t without a
 * session.  The split-K partial tiles and arrival counters live in a static
 * device array of 16 MiB + 64 KiB per GPU, held until the process ends.  The
 * kernel (chosen by M as for cpq_affine_qmm_t) is the one a default session
 * runs whenever its K split fits that array (then the result is
 * bit-identical); otherwise the best plan for the
 * array's capacity (a smaller split or none: same tolerance, another
 * summation order).  The stream must belong to a device of this process (the
 * current device for the null stream); the array of that device is used.  It
 * calls no allocator.  Calls that overlap on one GPU (two streams or
 * threads) share that array and race: serialise them. */
cpq_status cpq_affine_qmm_t_noalloc(void* hip_stream, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                                    const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                                    const void* x, size_t x_len, void* y, size_t y_len, size_t m, size_t n,
                                    size_t k, uint32_t group_size, uint32_t bits);

/* affine_dequantize_bf16_gs64_b4 (dequantize.rs:58-137), any (T, gs, bits):
 * out[i] = RNE_T(fmaf(scale, q_i, bias)) for out_len elements laid out as
 * consecutive groups of group_size.  out_len == 0 is a no-op. */
cpq_status cpq_affine_dequantize(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                                 size_t w_q_len, const void* scales, size_t scales_len,
                                 const void* biases, size_t biases_len, void* out,
                                 size_t out_len, uint32_t group_size, uint32_t bits);

/* Routed-expert quantized matmul.  No wired counterpart in the reference: its
 * semantics follow the vendored MSL affine_gather_qmm_t / affine_gather_qmm_rhs
 * (kernels-mlx/.../quantized.h:2092-2172, 2242-2436):
 *   Y[r, :] = X[lhs_indices[r], :] . dequant(W[rhs_indices[r]])^T,  r < n_rows.
 * W holds n_experts matrices of [N, K] back to back (scales/biases likewise).
 * lhs_indices may be NULL (row r reads X row r; X then has n_rows rows).
 * rhs_indices need not be sorted; sorted_indices=1 promises ascending order
 * (enables the run-walking schedule of gather_qmm_rhs).  Every index is
 * checked on the device: out-of-range entries produce a zero row and the
 * count of such rows is reported by the next cpq_commands_wait as
 * CPQ_ERR_INVALID_ARGUMENT. */
cpq_status cpq_affine_gather_qmm(cpq_commands* cmds, cpq_dtype dtype, const void* x,
                                 size_t x_rows, const uint32_t* w_q, size_t w_q_len,
                                 const void* scales, size_t scales_len, const void* biases,
                                 size_t biases_len, const uint32_t* lhs_indices,
                                 const uint32_t* rhs_indices, size_t n_rows, void* y,
                                 size_t y_len, size_t n_experts, size_t n, size_t k,
                                 uint32_t group_size, uint32_t bits, int sorted_indices);

/* dispatch_quantized_matmul (runtime/src/eval.rs:1293-1394): Y[M,N] for an
 * activation of M rows against a [N, k_physical] weight; routes by M to the
 * decode (M==1), small-batch, or prefill kernel.  x_len is the activation's
 * logical element count and x_alloc_bytes its allocation: M==1 follows the
 * qmv contract (K-padded activations allowed when the allocation covers
 * k_physical), M>1 the qmm_t contract (x_len == M*k_physical, N % 32 == 0). */
cpq_status cpq_quantized_matmul(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                                size_t w_q_len, const void* scales, size_t scales_len,
                                const void* biases, size_t biases_len, const void* x, size_t x_len,
                                size_t x_alloc_bytes, void* y, size_t m, size_t n,
                                size_t k_physical, uint32_t group_size, uint32_t bits);

/* Host-only argument validators used by the ops above (callable without a GPU). */
cpq_status cpq_check_qmv_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                              size_t biases_len, size_t x_alloc_bytes, size_t y_len,
                              size_t in_vec_size, uint32_t group_size, uint32_t bits);
cpq_status cpq_check_qmm_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                              size_t biases_len, size_t x_len, size_t y_len, size_t m, size_t n,
                              size_t k, uint32_t group_size, uint32_t bits);
cpq_status cpq_check_dequantize_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                                     size_t biases_len, size_t out_len, uint32_t group_size,
                                     uint32_t bits);
cpq_status cpq_check_embed_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len, size_t biases_len,
                                size_t n_ids, size_t vocab, size_t hidden, size_t out_len,
                                uint32_t group_size, uint32_t bits);
cpq_status cpq_check_gather_args(cpq_dtype dtype, size_t x_rows, size_t w_q_len,
                                 size_t scales_len, size_t biases_len, int has_lhs,
                                 size_t n_rows, size_t y_len, size_t n_experts, size_t n,
                                 size_t k, uint32_t group_size, uint32_t bits);

/* Batched qmv / qmm_t (MLX's `batched` kernel variants; adjust_matrix_offsets,
 * quantized.h:1351-1388): over batch_shape[batch_ndims] (row-major), element z
 * takes its W, scales, biases and x at the given element strides (u32 words
 * for w_q, T elements otherwise; stride 0 broadcasts), and writes its
 * [M, N] (qmv: [N]) block of y contiguously at z*M*N.  Each element's matrix
 * must lie inside its buffer; w_q strides must be multiples of 4 words and x
 * strides of 8 elements.  Encode only: weights shared by every element with
 * dense activations run as one matmul over all rows; otherwise the decode
 * kernels take the batch in a grid dimension where the shape allows, else
 * each element is one single-matrix launch on the session stream. */
cpq_status cpq_affine_qmm_t_batched(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                                    const void* scales, size_t scales_len, const void* biases,
                                    size_t biases_len, const void* x, size_t x_len, void* y, size_t y_len,
                                    size_t m, size_t n, size_t k, uint32_t group_size, uint32_t bits,
                                    int batch_ndims, const int* batch_shape, const int64_t* w_strides,
                                    const int64_t* s_strides, const int64_t* b_strides,
                                    const int64_t* x_strides);
cpq_status cpq_affine_qmv_batched(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                                  const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                                  const void* x, size_t x_len, void* y, size_t y_len, size_t n, size_t k,
                                  uint32_t group_size, uint32_t bits, int batch_ndims, const int* batch_shape,
                                  const int64_t* w_strides, const int64_t* s_strides, const int64_t* b_strides,
                                  const int64_t* x_strides);

/* affine_qmm_n / affine_qvm (MLX transpose=false; quantized.h:977-1086,
 * 1215-1349): Y[M, N] = X[M, K] . dequant(W) with W logically [K, N] --
 * w_q [K, N*bits/32] packed along N, scales / biases [K, N/group_size].
 * qvm is the M == 1 case.  Same numerics contract as cpq_affine_qmm_t.
 * N % 32 == 0 and K % 8 == 0.  The reference's runtime rejects
 * transpose=false (tensor.rs:2069-2075), so cpq_quantized_matmul and the
 * graph node do too; this is the kernels-level op. */
cpq_status cpq_check_qmm_n_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len, size_t biases_len,
                                size_t x_len, size_t y_len, size_t m, size_t n, size_t k,
                                uint32_t group_size, uint32_t bits);
cpq_status cpq_affine_qmm_n(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                            const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                            const void* x, size_t x_len, void* y, size_t y_len, size_t m, size_t n, size_t k,
                            uint32_t group_size, uint32_t bits);

/* embed_tokens (cider-press-models/src/nn.rs:123-136): out[t, :] =
 * dequantize(W[ids[t], :]) for a quantized [vocab, hidden] table, T out.
 * The reference gathers the packed words, scales and biases
 * (Tensor::gather, runtime/src/tensor.rs:1444-1530) and dequantizes the
 * gathered triple; here one kernel does both, bit-identical to that.
 * ids (device, U32, n_ids) at or past vocab give zero rows and are reported
 * by the next cpq_commands_wait as CPQ_ERR_INVALID_ARGUMENT. */
cpq_status cpq_embed_tokens(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                            const void* scales, size_t scales_len, const void* biases,
                            size_t biases_len, const uint32_t* ids, size_t n_ids, size_t vocab,
                            size_t hidden, void* out, size_t out_len, uint32_t group_size,
                            uint32_t bits);

/* Routed experts around cpq_affine_gather_qmm.  No reference counterpart:
 * the reference names the router, top-k selection and the gather_qmm feed as
 * its unbuilt MoE feature (docs/inference/feed-forward.md:98-107, 131-137).
 *
 * moe_route: per token t, p = softmax(logits[t, :]) in fp32 (logits F32,
 * F16 or BF16, [tokens, n_experts]); experts[t*k + j] / scores[t*k + j] are
 * the k largest p in descending order (ties: lower expert first), divided by
 * their sum when `normalize`.  Then the rows r = t*k + j are sorted by
 * expert, stably: lhs[p] = token and rhs[p] = expert of sorted row p (the
 * sorted-index inputs of cpq_affine_gather_qmm), inv[r] = sorted position
 * of row r, offsets[e] = first sorted row of expert e, offsets[E] = tokens*k.
 * n_experts <= 1024, top_k <= min(16, n_experts).  Uses session scratch. */
cpq_status cpq_moe_route(cpq_commands* cmds, cpq_dtype logits_dtype, const void* logits, size_t tokens,
                         size_t n_experts, uint32_t top_k, int normalize, uint32_t* experts, float* scores,
                         uint32_t* lhs, uint32_t* rhs, uint32_t* inv, uint32_t* offsets);
/* moe_combine: out[t, :] = RNE_T(sum_j scores[t*k + j] * y[inv[t*k + j], :]),
 * fp32 accumulation in j order; y is the [tokens*k, N] expert output in
 * sorted row order.  A position outside the rows contributes nothing and is
 * reported by the next wait as CPQ_ERR_INVALID_ARGUMENT. */
cpq_status cpq_moe_combine(cpq_commands* cmds, cpq_dtype dtype, const void* y, size_t y_len, const float* scores,
                           const uint32_t* inv, size_t tokens, uint32_t top_k, size_t n, void* out,
                           size_t out_len);

/* ------------------------------------------------------------------ */
/* Runtime node (runtime/src/{quantized,tensor,eval}.rs)                 */
/* ------------------------------------------------------------------ */

/* QuantizedWeight::from_bytes / from_bytes_k_padded (quantized.rs:59-125):
 * logical shape [n, k_logical] stored as physical [n, k_physical];
 * k_logical == k_physical for an unpadded weight.  Byte lengths are checked. */
cpq_status cpq_qweight_from_bytes(cpq_device* dev, cpq_dtype dtype, size_t n,
                                  size_t k_physical, size_t k_logical, uint32_t bits,
                                  uint32_t group_size, const void* weights, size_t weights_bytes,
                                  const void* scales, size_t scales_bytes, const void* biases,
                                  size_t biases_bytes, cpq_qweight** out);
void cpq_qweight_release(cpq_qweight* w);

/* A dense leaf tensor uploaded from host memory (contiguous, row-major):
 * BF16 / F16 activations, or U32 token ids. */
cpq_status cpq_tensor_from_host(cpq_device* dev, cpq_dtype dtype, const size_t* dims,
                                size_t ndim, const void* data, cpq_tensor** out);
/* Tensor::quantized_matmul (tensor.rs:2064-2171): records a lazy
 * QuantizedMatMul node; no GPU work.  transpose must be 1. */
cpq_status cpq_tensor_quantized_matmul(cpq_tensor* x, cpq_qweight* w, int transpose,
                                       cpq_tensor** out);
/* Tensor::dequantize_affine (tensor.rs:1558-1637): lazy Dequantize node producing
 * the dense [n, k_physical] weight. */
cpq_status cpq_tensor_dequantize(cpq_qweight* w, cpq_tensor** out);
/* embed_tokens (nn.rs:123-136) as a lazy node: rank-1 U32 ids against an
 * unpadded [vocab, hidden] weight; the result is [n_ids, hidden] of the
 * weight's T. */
cpq_status cpq_tensor_embed_tokens(cpq_tensor* ids, cpq_qweight* w, cpq_tensor** out);
/* Tensor::eval (tensor.rs:2681): encodes every pending node on the device's
 * session, commits and waits. */
cpq_status cpq_tensor_eval(cpq_tensor* t);
cpq_status cpq_tensor_shape(cpq_tensor* t, size_t* dims, size_t cap, size_t* ndim);
/* Host copy of an evaluated tensor (Tensor::cpu_slice). */
cpq_status cpq_tensor_read(cpq_tensor* t, void* host, size_t byte_len);
void cpq_tensor_release(cpq_tensor* t);

/* QuantizedWeight accessors: logical / physical shape, quantization, T. */
cpq_status cpq_qweight_info(const cpq_qweight* w, size_t* n, size_t* k_physical, size_t* k_logical,
                            uint32_t* bits, uint32_t* group_size, cpq_dtype* dtype);

/* ------------------------------------------------------------------ */
/* On-disk format: MLX-style safetensors archives                        */
/* (cider-press-models/src/safetensors_io.rs, qwen2/{weights,config}.rs) */
/* ------------------------------------------------------------------ */

/* safetensors::SafeTensors analogue.  open() maps the file read-only
 * (tensor bytes are uploaded from the mapping); deserialize() copies an
 * in-memory archive.  A malformed header, an unknown dtype, a byte size that
 * does not match dtype x shape, or entries that do not tile the byte buffer
 * return CPQ_ERR_SAFETENSORS. */
typedef struct cpq_safetensors cpq_safetensors;
cpq_status cpq_safetensors_open(const char* path, cpq_safetensors** out);
cpq_status cpq_safetensors_deserialize(const void* bytes, size_t len, cpq_safetensors** out);
void cpq_safetensors_close(cpq_safetensors* st);
/* Tensor names, sorted. */
cpq_status cpq_safetensors_len(const cpq_safetensors* st, size_t* n);
cpq_status cpq_safetensors_name(const cpq_safetensors* st, size_t i, const char** name);
/* SafeTensors::tensor: dtype name ("U32", "BF16", ...), shape, and a view of
 * the bytes (valid until close).  CPQ_ERR_MISSING_KEY if absent. */
cpq_status cpq_safetensors_tensor(const cpq_safetensors* st, const char* key, const char** dtype,
                                  size_t* dims, size_t cap, size_t* ndim, const void** data,
                                  size_t* nbytes);
/* "__metadata__" string entries; CPQ_ERR_MISSING_KEY if absent. */
cpq_status cpq_safetensors_metadata(const cpq_safetensors* st, const char* key, const char** value);

/* read_quantized_weight (safetensors_io.rs:43-134): the triple
 * {base}.weight (U32 [N, K*bits/32]), {base}.scales and {base}.biases
 * ([N, K/group_size], BF16 -- or F16, both alike) into a QuantizedWeight of
 * logical shape [N, K].  Checks in the reference's order: MissingKey,
 * UnsupportedDtype, rank / packed-K / group divisibility (InvalidArgument),
 * then ShapeMismatch of scales and biases.  The archive is checked before the
 * device is touched. */
cpq_status cpq_read_quantized_weight(cpq_device* dev, const cpq_safetensors* st, const char* base_name,
                                     uint32_t bits, uint32_t group_size, cpq_qweight** out);
/* build_padded_twin (qwen2/weights.rs:297-307): the same triple, zero-padded
 * along K to k_pad (>= K, a multiple of group_size) with zero words, scales
 * and biases; logical K stays K. */
cpq_status cpq_read_quantized_weight_k_padded(cpq_device* dev, const cpq_safetensors* st,
                                              const char* base_name, uint32_t bits,
                                              uint32_t group_size, size_t k_pad, cpq_qweight** out);
/* pad_quantized_k (qwen2/weights.rs:316-376) on host bytes: rows of
 * k*bits/8 packed bytes and (k/gs) 16-bit scales/biases widened to k_pad;
 * outputs are caller-allocated ([n * k_pad*bits/8], [n * (k_pad/gs) * 2]). */
cpq_status cpq_pad_quantized_k(const void* weights, const void* scales, const void* biases, size_t n,
                               size_t k, size_t k_pad, uint32_t bits, uint32_t group_size,
                               size_t sb_elem_bytes, void* w_out, void* s_out, void* b_out);
/* read_dense_tensor (safetensors_io.rs:25-32) for the graph's element types
 * (BF16, F16); other dtypes return CPQ_ERR_UNSUPPORTED_DTYPE. */
cpq_status cpq_read_dense_tensor(cpq_device* dev, const cpq_safetensors* st, const char* key,
                                 cpq_tensor** out);
/* The "quantization": {"group_size", "bits"} block of config.json
 * (qwen2/config.rs:65-73).  *present = 0 when the key is absent or null;
 * malformed JSON or wrongly typed fields return CPQ_ERR_JSON. */
cpq_status cpq_quantization_from_config(const char* json, size_t len, int* present, uint32_t* bits,
                                        uint32_t* group_size);

#ifdef __cplusplus
}
#endif

#endif /* CPQ_H */
