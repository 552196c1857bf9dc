// Internal declarations shared by the host runtime, the op dispatchers and
// the HIP kernel launchers of libcpq.so.  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <cstdlib>
#include <string>
#include <vector>

#include "../../include/cpq.h"

struct cpq_device {
  int ordinal = 0;
  int cu_count = 0;
  int clock_khz = 0;
  int xcd_count = 8;
  char name[256] = {0};
  // Session used by Tensor::eval (created on first use, released with the device).
  struct cpq_commands* eval_session = nullptr;
};

struct cpq_commands {
  cpq_device* dev = nullptr;
  hipStream_t stream = nullptr;
  bool owns_stream = false;
  // Device-side status words: kernels that can detect bad data count it
  // here ([0] gather rows with out-of-range indices, [1] embed ids out of
  // range, [2] MoE combine positions out of range)
  // add to it; cpq_commands_wait reads and clears it.
  unsigned int* status = nullptr;
  // Scratch of the split-K reductions and the routing sort: arrival
  // counters (zero between launches) followed by fp32 partial tiles or sort
  // histograms.  Allocated once when the session is made, with a fixed
  // capacity; ops never grow it (kernel selection must not depend on graph
  // capture, during which nothing can be allocated).
  void* scratch = nullptr;
  size_t scratch_bytes = 0;
  // Per-op GPU timing of a profiled session (cpq_commands_create_profiled):
  // two timing events per op of capacity, created with the session; the
  // index of the next unused one; per recorded op its label and the indices
  // of its start and end events; whether the last op is still open (its end
  // not yet recorded).  Empty for an ordinary session.
  struct ProfiledOp {
    std::string label;
    size_t start = 0, end = 0;
  };
  bool profiled = false;
  std::vector<hipEvent_t> prof_events;
  size_t prof_cursor = 0;
  std::vector<ProfiledOp> prof_ops;
  bool prof_open = false;
  // Labels of the last resolved batch; cpq_gpu_segment.label points here.
  std::vector<std::string> prof_resolved_labels;
};

struct cpq_event {
  hipEvent_t ev = nullptr;
};

struct cpq_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};

namespace cpq {

// Per-thread error text (cpq_last_error_message).
cpq_status fail(cpq_status st, const std::string& msg);
cpq_status hip_fail(hipError_t e, const char* what);

inline size_t dtype_size(cpq_dtype t) { return t == CPQ_DTYPE_F32 || t == CPQ_DTYPE_U32 ? 4 : 2; }

bool kernel_available(cpq_dtype dtype, uint32_t group_size, uint32_t bits);

// ---------------------------------------------------------------------------
// Kernel launchers (defined in kernels/*.hip).  Shapes are validated by the
// callers; launchers only assert the invariants their grids rely on.
// ---------------------------------------------------------------------------

struct QuantArgs {
  const uint32_t* w;   // [rows, K*bits/32] (per expert for gather)
  const void* scales;  // [rows, K/gs]
  const void* biases;  // [rows, K/gs]
  int gs;
  int bits;
  cpq_dtype dtype;
};

hipError_t launch_dequantize(hipStream_t s, const QuantArgs& q, void* out, size_t n_out);
// Y[M, N] = X[M, K] . dequant(W[K, N]) (MLX transpose=false); N % 32 == 0,
// K % 8 == 0.  split > 1 splits K and needs qmm_n_scratch_bytes of fp32 partials.
int qmm_n_split(int m, int n, int k, int cu_count);
size_t qmm_n_scratch_bytes(int m, int n, int split);
hipError_t launch_qmm_n(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                        float* partial);
// Decode (M = 1) transpose=false at 4/8 bits on the VALU: rows per thread
// and step, K parts and the split-K scratch they need (arrival words at the
// head, zero between launches, then fp32 sums); parts == 1 needs none.
// qvm_plan never asks for more than scratch_cap.
bool qvm_fits(const QuantArgs& q, int n, int k);
struct QvmPlan {
  int rpt;
  int parts;
  int k_part;
  size_t scratch_bytes;
};
QvmPlan qvm_plan(const QuantArgs& q, int n, int k, int cu_count, size_t scratch_cap);
hipError_t launch_qvm(hipStream_t s, const QvmPlan& p, void* scratch, const QuantArgs& q, const void* x, void* y,
                      int n, int k);
// Routed-expert plumbing (kernels/moe.hip): top-k routing, stable sort of
// (token, slot) rows by expert, weighted combine back to tokens.
size_t moe_sort_scratch_bytes(int rows, int n_experts);
hipError_t launch_moe_route(hipStream_t s, int logits_dtype, const void* logits, int tokens, int n_experts, int top_k,
                            int normalize, uint32_t* experts, float* scores);
hipError_t launch_moe_sort(hipStream_t s, const uint32_t* experts, int rows, int top_k, int n_experts,
                           uint32_t* scratch, uint32_t* lhs, uint32_t* rhs, uint32_t* inv, uint32_t* offsets);
hipError_t launch_moe_combine(hipStream_t s, int dtype, const void* y, const float* scores, const uint32_t* inv,
                              int tokens, int top_k, int n, void* out, unsigned int* bad);

// Rows ids[t] of a [vocab, hidden] table, dequantized into out[t, :]; ids at
// or past vocab give zero rows and are counted in *bad.
hipError_t launch_embed(hipStream_t s, const QuantArgs& q, const uint32_t* ids, uint32_t n_ids, uint32_t vocab,
                        uint32_t hidden, void* out, unsigned int* bad);

// Decode GEMV: y[N] = x[K] . W^T for one activation row.
hipError_t launch_qmv(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k);

// A batch folded into a grid dimension (MLX's adjust_matrix_offsets):
// element z (row-major over shape[0..nd)) takes its operands at
// sum_d idx_d(z) * st[o][d] elements (o: w_q in u32 words, scales, biases,
// x in T elements) and writes its output block at z * (block size).
constexpr int kMaxBatchDims = 8;
struct BatchArgs {
  int nd;
  int shape[kMaxBatchDims];
  long long st[4][kMaxBatchDims];
};
// The decode kernel with the batch in its grid (4/8-bit, gs 32/64/128,
// K a multiple of 2048 up to 16384; every element's scales and biases
// 8-byte aligned): whether it takes the shape, and the launch.
bool qmv_batch_fits(const QuantArgs& q, int n, int k);
hipError_t launch_qmv_batched(hipStream_t s, const QuantArgs& q, const void* x, void* y, int n, int k, int count,
                              const BatchArgs& ba);
// The decode layout for up to 16 rows with the batch in its grid (shape
// limits of qmv_rows_fits, for every element).
hipError_t launch_qmv_rows_batched(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                                   int count, const BatchArgs& ba);
// The decode layout for up to 16 rows: Y[M, N] = X[M, K] . W^T (shape limits
// in qmv_rows_fits).
bool qmv_rows_fits(const QuantArgs& q, int m, int n, int k, const void* x);
hipError_t launch_qmv_rows(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k);

// Small-M GEMM on the matrix cores with VALU dequantization (M rows, any M;
// processed 16 rows at a time).  Also the gather kernel body.
hipError_t launch_qmm_skinny(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m,
                             int n, int k);

// Prefill GEMM.  qmm_plan picks the kernel (and its K split) from the shape,
// the CU count and the capacity of the scratch the caller can give it;
// launch_qmm runs that plan, with `scratch` holding at least
// plan.scratch_bytes (arrival counters zeroed) when that is nonzero.
enum class QmmKernel { Unsplit, Wide, Dma };
struct QmmPlan {
  QmmKernel kernel;      // Dma / Wide (4-bit, K split possible) or a kernel that needs no scratch
  int split;             // its K split
  size_t scratch_bytes;  // scratch the plan uses (0: none)
};
QmmPlan qmm_plan(const QuantArgs& q, int m, int n, int k, int cu_count, size_t scratch_cap);
hipError_t launch_qmm(hipStream_t s, const QmmPlan& plan, void* scratch, const QuantArgs& q, const void* x,
                      void* y, int m, int n, int k);

// qmm_plan + launch_qmm on a session (its stream, CU count and scratch).
hipError_t launch_session_qmm(cpq_commands* cmds, const QuantArgs& q, const void* x, void* y, int m, int n, int k);

// Where a matmul runs: stream, CU count, the split-K scratch at hand and the
// capacity plans are made for (plans needing more than scratch_bytes are
// remade for scratch_bytes).
struct ExecCtx {
  hipStream_t stream;
  int cu_count;
  void* scratch;
  size_t plan_bytes;
  size_t scratch_bytes;
};
ExecCtx session_ctx(const cpq_commands* cmds);
// Y = X . W^T with the kernel chosen by M (small-M kernels, else the prefill
// plan), as affine_qmm_t and the runtime node run it.
hipError_t launch_matmul(const ExecCtx& ex, const QuantArgs& q, const void* x, void* y, int m, int n, int k);

// Capacity of a session's scratch when CPQ_SESSION_SCRATCH_MB is not set.
constexpr size_t kDefaultSessionScratchBytes = size_t(64) << 20;

// Prefill kernels that need no session scratch (staged, streaming or the
// LDS-tiled fallback, by shape); any M, K, group size and width.
hipError_t launch_qmm_unsplit(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k);

// Wide-tile prefill kernel (4-bit, 128 x 128 tiles, optional split K).
constexpr size_t kWideCounterBytes = 64 * 1024;  // arrival counters at the head of the scratch
bool qmm_wide_fits(int m, int n, int k, int gs, int bits, int split);
// Split (1, 2 or 4) that minimises the estimated makespan; 0 if the kernel
// does not apply.
int qmm_wide_split(int m, int n, int k, int gs, int bits, int cu_count);
size_t qmm_wide_scratch_bytes(int m, int n, int split);
hipError_t launch_qmm_wide(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n,
                           int k, int split, void* scratch);
hipError_t zero_words(hipStream_t s, void* p, size_t n_words);

// Prefill kernel with two waves per SIMD (4-bit, 128 x 128 tiles, both
// operands streamed into LDS, optional split K; same scratch layout as the
// wide kernel: arrival counters, then fp32 partial tiles).
bool qmm_dma_fits(int m, int n, int k, int gs, int bits, int split);
int qmm_dma_split(int m, int n, int k, int gs, int bits, int cu_count);
size_t qmm_dma_scratch_bytes(int m, int n, int split);
hipError_t launch_qmm_dma(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k, int split,
                          void* scratch);

// The session's scratch when it holds at least `bytes` (counters zeroed):
// true and *out set, else false.  Depends on the session's fixed capacity
// only, so a kernel choice made from it is the same eagerly and under graph
// capture.
bool session_scratch(const cpq_commands* cmds, size_t bytes, void** out);

// Routed experts, expert-major kernel (4/8-bit, K % 128 == 0): one
// workgroup per (expert, column chunk); it also validates the indices (bad
// rows zeroed, bad rows and sorted-order descents counted into *status).  gather_expert_supported says whether
// it applies; launch_gather_qmm uses it when it does.
bool gather_expert_supported(int bits, int x_rows, int n_rows, int n, int k);
hipError_t launch_gather_expert(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                                const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                                int n_experts, int n, int k, bool sorted, int cu_count,
                                unsigned int* status);

// Routed experts at decode shapes (kernels/gather_decode.hip): up to 64
// rows, 4/8-bit, K % 128 == 0; one workgroup per (distinct expert, 16
// columns); validates the indices itself.
int gather_decode_kw(int slots, int n, int k, bool dense);
size_t gather_decode_lds(int rows_max, int k, int kw);
// The same kernel as a small-M matmul (rows in passes of 8, one workgroup
// per (column group, pass)): 1 <= M <= 64, 4/8-bit, K a multiple of the
// group size (a partial last 128-step is masked).  pad_exact: K split over
// 4 waves or 1 (never 2), so that zero K-padding to the next multiple of 512
// (zero weights, scales, biases and activations past the logical K) keeps
// every wave's steps and leaves every output bit unchanged.
bool dense_small_supported(const QuantArgs& q, int m, int n, int k);
hipError_t launch_dense_small(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                              bool pad_exact = false);
// Small-M kernel with the activation rows resident in LDS
// (kernels/qmm_rows.hip): 1 <= M <= 64, M * K * 2 <= 78 KiB, 4/8-bit,
// K % 128 == 0; one workgroup per 128 columns.
bool qmm_rows_supported(const QuantArgs& q, int m, int n, int k);
int qmm_rows_workgroups(int n);
hipError_t launch_qmm_rows(hipStream_t s, const QuantArgs& q, const void* x, void* y, int m, int n, int k);
bool gather_decode_supported(const QuantArgs& q, int x_rows, int n_rows, int n, int k);
hipError_t launch_gather_decode(hipStream_t s, const QuantArgs& q, const void* x, int x_rows, const uint32_t* lhs,
                                const uint32_t* rhs, int n_rows, void* y, int n_experts, int n, int k, bool sorted,
                                unsigned int* status);

// Whether some routed-expert kernel takes this shape: the expert-major
// kernel, or the per-slab kernel while its slab constants fit in LDS.
bool gather_supported(int bits, int n_rows, int n, int k, int gs);

// Routed experts.
hipError_t launch_gather_qmm(hipStream_t s, const QuantArgs& q, const void* x, int x_rows,
                             const uint32_t* lhs, const uint32_t* rhs, int n_rows, void* y,
                             int n_experts, int n, int k, bool sorted, unsigned int* status);

// Whether the small-M kernel's per-slab constants fit in LDS at this K and
// group size (16 columns x (K/gs + 1) x 16 bytes next to its static LDS).
bool skinny_fits(int k, int gs);

// Small-M kernel (kernels/qmm_small.hip), 1 <= M <= 64 at 4 and 8 bits, K a
// multiple of 256: K parts per column tile, chunks per part, K elements per
// chunk, 16-row blocks (the tile is 16*mb columns) and the split-K scratch it
// needs.  split == 0: the shape is not supported (or its split would need
// more scratch than scratch_cap).
struct SmallPlan {
  int split;
  int nch;
  int kb;
  int mb;
  size_t scratch_bytes;
};
SmallPlan qmm_small_plan(const QuantArgs& q, int m, int n, int k, int cu_count, size_t scratch_cap);
hipError_t launch_qmm_small(hipStream_t s, const SmallPlan& p, void* scratch, const QuantArgs& q, const void* x,
                            void* y, int m, int n, int k);

// Row-count threshold below which cpq_quantized_matmul uses the skinny kernel.
int skinny_max_m(const QuantArgs& q, int n, int k);

// Plain streaming read of up to 4 regions (measurement support), in one of
// stream_read_variant_count() designs.
hipError_t launch_stream_read(hipStream_t s, const void* const* regions, const size_t* bytes, int n_regions,
                              uint32_t* sink, int n_wg, int variant);
int stream_read_variant_count();

// Integer from the environment (tuning and test hooks), dflt when unset.
inline int env_int(const char* name, int dflt) {
  const char* e = std::getenv(name);
  return e && *e ? std::atoi(e) : dflt;
}

}  // namespace cpq
