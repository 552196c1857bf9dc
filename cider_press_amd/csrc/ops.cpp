// Op entry points of libcpq.so: argument validation, kernel selection, launch.
//
// Host-side mirror of the reference's typed dispatch functions:
//   crates/cider-press-kernels/src/kernels/qmv.rs:77-205         -> cpq_affine_qmv
//   crates/cider-press-kernels/src/kernels/qmm.rs:66-220         -> cpq_affine_qmm_t
//   crates/cider-press-kernels/src/kernels/dequantize.rs:58-137  -> cpq_affine_dequantize
//   crates/cider-press-runtime/src/eval.rs:1293-1394             -> cpq_quantized_matmul
// Validation order and messages follow those functions so error behaviour is
// the same; "kernel not found" is reported after shape validation, as the
// reference's pipeline lookup is (qmv.rs:172-173, library.rs:264-286).
#include <climits>
#include <cstdlib>
#include <string>

#include "cpq_internal.hpp"

namespace cpq {

bool kernel_available(cpq_dtype dtype, uint32_t group_size, uint32_t bits) {
  const bool t_ok = dtype == CPQ_DTYPE_BF16 || dtype == CPQ_DTYPE_F16;
  const bool gs_ok = group_size == 32 || group_size == 64 || group_size == 128;
  const bool b_ok = bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8;
  return t_ok && gs_ok && b_ok;
}

// Largest M the routed op sends to the small-M kernels (the decode layout for
// up to 16 rows, the tiled small-M kernel, or the slab kernel; see
// cpq_quantized_matmul).  Up to 32 rows they always win; at 33..64 rows they
// win while the prefill kernel's 128-wide tiles leave most CUs idle (N <=
// 8192) and lose once N fills the chip (slab kernel 58 vs 31 us at N =
// 12288).  CPQ_SKINNY_MAX_M overrides it, read once per process.  Shapes
// whose slab constants do not fit in LDS (K / gs beyond about 500 groups per
// row) never take them.
int skinny_max_m(const QuantArgs& q, int n, int k) {
  if (!skinny_fits(k, (int)q.gs)) return 0;  // its slab constants would not fit in LDS
  const int lim = env_int("CPQ_SKINNY_MAX_M", 0);  // tuning and test hook
  if (lim > 0) return lim;
  return n <= 8192 ? 64 : 32;
}

namespace {

const char* tname(cpq_dtype t) {
  return t == CPQ_DTYPE_BF16 ? "bfloat16_t" : t == CPQ_DTYPE_F16 ? "float16_t" : "float";
}

std::string kname(const char* op, cpq_dtype t, uint32_t gs, uint32_t bits) {
  return std::string("affine_") + op + "_" + tname(t) + "_gs_" + std::to_string(gs) + "_b_" +
         std::to_string(bits);
}

cpq_status not_found(const char* op, cpq_dtype t, uint32_t gs, uint32_t bits) {
  return fail(CPQ_ERR_KERNEL_NOT_FOUND, "kernel `" + kname(op, t, gs, bits) + "` not found in library");
}

cpq_status launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return hip_fail(e, what);
  return CPQ_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// The prefill op on a session: its stream, CU count and fixed-capacity scratch.
hipError_t launch_session_qmm(cpq_commands* cmds, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  const QmmPlan plan = qmm_plan(q, m, n, k, cmds->dev ? cmds->dev->cu_count : 0, cmds->scratch ? cmds->scratch_bytes : 0);
  return launch_qmm(cmds->stream, plan, cmds->scratch, q, x, y, m, n, k);
}

namespace {
bool aligned2(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1u) == 0; }

cpq_status check_ptrs(const char* op, const void* w, const void* s, const void* b, const void* x,
                      const void* y) {
  if (!w || !s || !b || !x || !y)
    return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": NULL buffer");
  if (!aligned16(w) || !aligned16(x) || !aligned16(y) || !aligned2(s) || !aligned2(b))
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                std::string(op) + ": w_q, x and y must be 16-byte aligned; scales/biases 2-byte");
  return CPQ_OK;
}

cpq_status check_dtype(const char* op, cpq_dtype t) {
  if (t != CPQ_DTYPE_F32 && t != CPQ_DTYPE_F16 && t != CPQ_DTYPE_BF16)
    return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": unknown dtype " + std::to_string(int(t)));
  return CPQ_OK;
}

// Checked a*b (size_t); false on overflow.
bool mul_ok(size_t a, size_t b, size_t* out) {
  if (a != 0 && b > SIZE_MAX / a) return false;
  *out = a * b;
  return true;
}

}  // namespace
}  // namespace cpq

using cpq::fail;

namespace cpq {

// Y[M, N] = X[M, K] . W^T on validated operands: the kernel the shape runs
// best on.  Up to skinny_max_m rows: at K = 4096 / 8192 / 16384 (4/8-bit, up
// to 16 rows) the decode kernel's layout with M activation rows; other
// 4/8-bit shapes with K a multiple of 256 the tiled small-M kernel; other
// shapes the slab kernel.  Larger M: the prefill plan.  Plans are made for
// ex.plan_bytes of scratch and, when that plan needs more than the
// ex.scratch_bytes at hand, for ex.scratch_bytes.  CPQ_SMALL_M=0 forces the
// slab kernel, CPQ_QMV_ROWS=0 skips the decode layout (tuning hooks).
hipError_t launch_matmul(const ExecCtx& ex, const QuantArgs& q, const void* x, void* y, int m, int n, int k) {
  // CPQ_SMALL_DENSE=1 forces the decode kernel's dense form where it
  // applies, 0 keeps it off (tuning hooks).
  const int dense_env = env_int("CPQ_SMALL_DENSE", -1);
  const bool dense_ok = dense_env != 0 && aligned16(x) && aligned16(q.w) && dense_small_supported(q, m, n, k);
  if (dense_ok && dense_env == 1) return launch_dense_small(ex.stream, q, x, y, m, n, k);
  // The LDS-resident small-M kernel (all rows of X in LDS, one workgroup
  // per 128 columns, each wave's loads in one batch up to K = 1024) where
  // it has a workgroup for every second CU at least: short K and large N,
  // such as a vocabulary projection at prefill.
  // CPQ_SMALL_ROWS=1 forces it where it applies, 0 keeps it off (tuning
  // hooks).
  const long cus = ex.cu_count > 0 ? ex.cu_count : 256;
  const int rows_env = env_int("CPQ_SMALL_ROWS", -1);
  const bool rows_ok = rows_env != 0 && aligned16(x) && aligned16(q.w) && qmm_rows_supported(q, m, n, k);
  if (rows_ok && (rows_env == 1 || (m >= 2 && k <= 1024 && 2L * qmm_rows_workgroups(n) >= cus)))
    return launch_qmm_rows(ex.stream, q, x, y, m, n, k);
  if (m <= skinny_max_m(q, n, k)) {
    const bool small_on = env_int("CPQ_SMALL_M", 1) != 0;
    const bool rows_on = env_int("CPQ_QMV_ROWS", 1) != 0;
    const bool words4 = ((reinterpret_cast<uintptr_t>(q.scales) | reinterpret_cast<uintptr_t>(q.biases)) & 3u) == 0;
    SmallPlan sp{0, 0, 0, 0, 0};
    if (small_on && aligned16(x) && aligned16(q.w) && words4) {
      sp = qmm_small_plan(q, m, n, k, ex.cu_count, ex.plan_bytes);
      if (sp.split > 0 && sp.scratch_bytes > ex.scratch_bytes)
        sp = qmm_small_plan(q, m, n, k, ex.cu_count, ex.scratch_bytes);
    }
    if (small_on && rows_on && qmv_rows_fits(q, m, n, k, x)) return launch_qmv_rows(ex.stream, q, x, y, m, n, k);
    // The tiled kernel where it has a workgroup for every fourth CU at
    // least; below that (few column tiles and a K that does not split), or
    // where its K granularity does not fit, the dense form of the decode
    // kernel (K in 128-element steps split over the waves of a workgroup,
    // 8 rows per workgroup).
    const long small_wgs = sp.split > 0 ? (long)sp.split * ((n + 16 * sp.mb - 1) / (16 * sp.mb)) : 0;
    if (dense_ok && small_wgs * 4 < cus) return launch_dense_small(ex.stream, q, x, y, m, n, k);
    if (sp.split > 0) return launch_qmm_small(ex.stream, sp, ex.scratch, q, x, y, m, n, k);
    return launch_qmm_skinny(ex.stream, q, x, y, m, n, k);
  }
  QmmPlan plan = qmm_plan(q, m, n, k, ex.cu_count, ex.plan_bytes);
  if (plan.scratch_bytes > ex.scratch_bytes) plan = qmm_plan(q, m, n, k, ex.cu_count, ex.scratch_bytes);
  return launch_qmm(ex.stream, plan, ex.scratch, q, x, y, m, n, k);
}

ExecCtx session_ctx(const cpq_commands* cmds) {
  const size_t cap = cmds->scratch ? cmds->scratch_bytes : 0;
  return ExecCtx{cmds->stream, cmds->dev ? cmds->dev->cu_count : 0, cmds->scratch, cap, cap};
}

namespace {

cpq_status route_matmul(cpq_commands* cmds, const QuantArgs& q, const void* x, void* y, int m, int n, int k,
                        const char* op) {
  const std::string what = std::string(op) + (m <= skinny_max_m(q, n, k) ? " (small-M) launch" : " (prefill) launch");
  return launched(launch_matmul(session_ctx(cmds), q, x, y, m, n, k), what.c_str());
}

}  // namespace
}  // namespace cpq

extern "C" {

// ---------------------------------------------------------------------------
// Validators
// ---------------------------------------------------------------------------

// qmv.rs:89-163
cpq_status cpq_check_qmv_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                              size_t biases_len, size_t x_alloc_bytes, size_t y_len,
                              size_t in_vec_size, uint32_t group_size, uint32_t bits) {
  cpq_status st = cpq::check_dtype("affine_qmv", dtype);
  if (st != CPQ_OK) return st;
  if (in_vec_size > (size_t)INT_MAX)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_qmv: K=" + std::to_string(in_vec_size) + " does not fit in i32");
  const size_t required = in_vec_size * cpq::dtype_size(dtype);
  if (x_alloc_bytes < required)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_qmv: activation allocation too small for K-padded read: alloc_len=" +
                    std::to_string(x_alloc_bytes) + " < required_bytes=" + std::to_string(required) +
                    " (K-padding requires capacity >= physical K * sizeof(T))");
  if (y_len > (size_t)INT_MAX)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_qmv: N=" + std::to_string(y_len) + " does not fit in i32");
  const long k = (long)in_vec_size, n = (long)y_len;
  if (k <= 0 || n <= 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: K (" + std::to_string(k) + ") and N (" +
                                              std::to_string(n) + ") must be positive");
  if (group_size == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: group_size must be positive");
  if ((size_t)k % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: K (" + std::to_string(k) +
                                              ") must be a multiple of group_size (" +
                                              std::to_string(group_size) + ")");
  const size_t groups_per_row = (size_t)k / group_size;
  const size_t expected_w_q = (size_t)n * (size_t)k * bits / 32;
  if (w_q_len != expected_w_q)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: w_q.len()=" + std::to_string(w_q_len) +
                                              " != N*K*bits/32 (" + std::to_string(expected_w_q) + ")");
  const size_t expected_groups = (size_t)n * groups_per_row;
  if (scales_len != expected_groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: scales.len()=" + std::to_string(scales_len) +
                                              " != N*K/group_size (" +
                                              std::to_string(expected_groups) + ")");
  if (biases_len != expected_groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: biases.len()=" + std::to_string(biases_len) +
                                              " != N*K/group_size (" +
                                              std::to_string(expected_groups) + ")");
  if (!cpq::kernel_available(dtype, group_size, bits))
    return cpq::not_found((((size_t)n % 8 == 0) && ((size_t)k % 512 == 0)) ? "qmv_fast" : "qmv",
                          dtype, group_size, bits);
  return CPQ_OK;
}

// qmm.rs:80-119 and validate_qmm_buffer_lens (qmm.rs:165-220)
cpq_status cpq_check_qmm_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                              size_t biases_len, size_t x_len, size_t y_len, size_t m, size_t n,
                              size_t k, uint32_t group_size, uint32_t bits) {
  cpq_status st = cpq::check_dtype("affine_qmm_t", dtype);
  if (st != CPQ_OK) return st;
  if (m > (size_t)INT_MAX)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: M=" + std::to_string(m) + " does not fit in i32");
  if (n > (size_t)INT_MAX)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: N=" + std::to_string(n) + " does not fit in i32");
  if (k > (size_t)INT_MAX)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: K=" + std::to_string(k) + " does not fit in i32");
  if (m == 0 || n == 0 || k == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: M (" + std::to_string(m) + "), N (" +
                                              std::to_string(n) + "), K (" + std::to_string(k) +
                                              ") must all be positive");
  if (group_size == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: group_size must be positive");
  if (k % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: K (" + std::to_string(k) +
                                              ") must be a multiple of group_size (" +
                                              std::to_string(group_size) + ")");
  if (n % 32 != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: N (" + std::to_string(n) +
                                              ") must be a multiple of 32 (aligned variant only)");
  size_t nk, nkb, groups, mk, mn;
  if (!cpq::mul_ok(n, k, &nk))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: N*K overflows usize");
  if (!cpq::mul_ok(nk, bits, &nkb))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: N*K*bits overflows usize");
  const size_t expected_w_q = nkb / 32;
  if (w_q_len != expected_w_q)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: w_q.len()=" + std::to_string(w_q_len) +
                                              " != N*K*bits/32 (" + std::to_string(expected_w_q) + ")");
  if (!cpq::mul_ok(n, k / group_size, &groups))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: N*(K/group_size) overflows usize");
  if (scales_len != groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: scales.len()=" + std::to_string(scales_len) +
                                              " != N*K/group_size (" + std::to_string(groups) + ")");
  if (biases_len != groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: biases.len()=" + std::to_string(biases_len) +
                                              " != N*K/group_size (" + std::to_string(groups) + ")");
  if (!cpq::mul_ok(m, k, &mk)) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: M*K overflows usize");
  if (x_len != mk)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: x.len()=" + std::to_string(x_len) +
                                              " != M*K (" + std::to_string(mk) + ")");
  if (!cpq::mul_ok(m, n, &mn)) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: M*N overflows usize");
  if (y_len != mn)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: y.len()=" + std::to_string(y_len) +
                                              " != M*N (" + std::to_string(mn) + ")");
  if (!cpq::kernel_available(dtype, group_size, bits))
    return cpq::not_found("qmm_t", dtype, group_size, bits);
  return CPQ_OK;
}

// dequantize.rs:66-104, generalised over (T, group_size, bits)
cpq_status cpq_check_dequantize_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len,
                                     size_t biases_len, size_t out_len, uint32_t group_size,
                                     uint32_t bits) {
  cpq_status st = cpq::check_dtype("affine_dequantize", dtype);
  if (st != CPQ_OK) return st;
  if (out_len == 0) return CPQ_OK;
  if (bits == 0 || bits > 8)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: bits " + std::to_string(bits) +
                                              " outside 1..=8");
  // Elements per packed unit (per byte for 2/4/8-bit, per 3- or 5-byte pack otherwise).
  const size_t pack_factor = (bits == 3 || bits == 5) ? 8 : (bits == 6 ? 4 : 8 / bits);
  if (out_len % pack_factor != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: out element count " +
                                              std::to_string(out_len) +
                                              " not a multiple of pack_factor " +
                                              std::to_string(pack_factor));
  if (group_size == 0 || out_len % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: out element count " +
                                              std::to_string(out_len) +
                                              " not a multiple of group_size " +
                                              std::to_string(group_size));
  const size_t groups = out_len / group_size;
  if (scales_len != groups || biases_len != groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: scales/biases length mismatch (expected " +
                                              std::to_string(groups) + ", got scales=" +
                                              std::to_string(scales_len) + ", biases=" +
                                              std::to_string(biases_len) + ")");
  size_t total_bits;
  if (!cpq::mul_ok(out_len, bits, &total_bits))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: out_len*bits overflows usize");
  const size_t expected = total_bits / 32;
  if (total_bits % 32 != 0 || w_q_len != expected)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: w_q length " + std::to_string(w_q_len) +
                                              " != expected uint32 count " + std::to_string(expected));
  if (!cpq::kernel_available(dtype, group_size, bits))
    return cpq::not_found("dequantize", dtype, group_size, bits);
  return CPQ_OK;
}

cpq_status cpq_check_gather_args(cpq_dtype dtype, size_t x_rows, size_t w_q_len,
                                 size_t scales_len, size_t biases_len, int has_lhs,
                                 size_t n_rows, size_t y_len, size_t n_experts, size_t n,
                                 size_t k, uint32_t group_size, uint32_t bits) {
  cpq_status st = cpq::check_dtype("affine_gather_qmm", dtype);
  if (st != CPQ_OK) return st;
  if (n_rows > (size_t)INT_MAX || x_rows > (size_t)INT_MAX || n > (size_t)INT_MAX ||
      k > (size_t)INT_MAX || n_experts > 65535)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_gather_qmm: n_rows, x_rows, N, K must fit in i32 and n_experts <= 65535");
  if (n == 0 || k == 0 || n_experts == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: N (" + std::to_string(n) + "), K (" +
                                              std::to_string(k) + ") and n_experts (" +
                                              std::to_string(n_experts) + ") must be positive");
  if (group_size == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: group_size must be positive");
  if (k % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: K (" + std::to_string(k) +
                                              ") must be a multiple of group_size (" +
                                              std::to_string(group_size) + ")");
  if (!has_lhs && x_rows != n_rows)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: without lhs_indices x must have n_rows (" +
                                              std::to_string(n_rows) + ") rows, got " +
                                              std::to_string(x_rows));
  size_t per_w, w_total, per_g, g_total, yn;
  if (!cpq::mul_ok(n, k, &per_w) || !cpq::mul_ok(per_w, bits, &per_w) ||
      !cpq::mul_ok(per_w / 32, n_experts, &w_total))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: n_experts*N*K*bits overflows usize");
  if (w_q_len != w_total)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: w_q.len()=" + std::to_string(w_q_len) +
                                              " != n_experts*N*K*bits/32 (" + std::to_string(w_total) + ")");
  if (!cpq::mul_ok(n, k / group_size, &per_g) || !cpq::mul_ok(per_g, n_experts, &g_total))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: group count overflows usize");
  if (scales_len != g_total || biases_len != g_total)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: scales/biases length mismatch (expected " +
                                              std::to_string(g_total) + ", got scales=" +
                                              std::to_string(scales_len) + ", biases=" +
                                              std::to_string(biases_len) + ")");
  if (!cpq::mul_ok(n_rows, n, &yn) || y_len != yn)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: y.len()=" + std::to_string(y_len) +
                                              " != n_rows*N (" + std::to_string(n_rows * n) + ")");
  if (!cpq::kernel_available(dtype, group_size, bits))
    return cpq::not_found("gather_qmm", dtype, group_size, bits);
  return CPQ_OK;
}

// nn.rs:123-136 preconditions, plus the table geometry a fused kernel needs.
cpq_status cpq_check_embed_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len, size_t biases_len,
                                size_t n_ids, size_t vocab, size_t hidden, size_t out_len, uint32_t group_size,
                                uint32_t bits) {
  cpq_status st = cpq::check_dtype("embed_tokens", dtype);
  if (st != CPQ_OK) return st;
  st = cpq_quantization_validate(bits, group_size);
  if (st != CPQ_OK) return st;
  if (vocab == 0 || hidden == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: table shape must be non-empty [vocab, hidden]");
  if (hidden % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: hidden=" + std::to_string(hidden) +
                                              " must be a multiple of group_size=" + std::to_string(group_size));
  size_t vh, words, groups, th;
  if (!cpq::mul_ok(vocab, hidden, &vh)) return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: vocab*hidden overflows");
  words = vh / 32 * bits;  // hidden % 32 == 0 (group sizes are >= 32)
  groups = vh / group_size;
  if (w_q_len != words)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: w_q.len()=" + std::to_string(w_q_len) + " != vocab*hidden*bits/32 (" +
                                              std::to_string(words) + ")");
  if (scales_len != groups || biases_len != groups)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: scales/biases length mismatch (expected " +
                                              std::to_string(groups) + ", got scales=" + std::to_string(scales_len) +
                                              ", biases=" + std::to_string(biases_len) + ")");
  if (!cpq::mul_ok(n_ids, hidden, &th) || out_len != th)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: out.len()=" + std::to_string(out_len) +
                                              " != n_ids*hidden (" + std::to_string(n_ids * hidden) + ")");
  if (vocab > 0xFFFFFFFFull || th / 32 >= (1ull << 31))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: vocab or n_ids*hidden/32 beyond 32-bit indexing");
  if (!cpq::kernel_available(dtype, group_size, bits)) return cpq::not_found("dequantize", dtype, group_size, bits);
  return CPQ_OK;
}

// qmm_n / qvm (transpose=false): W is [K, N] packed along N, groups along N.
cpq_status cpq_check_qmm_n_args(cpq_dtype dtype, size_t w_q_len, size_t scales_len, size_t biases_len,
                                size_t x_len, size_t y_len, size_t m, size_t n, size_t k, uint32_t group_size,
                                uint32_t bits) {
  cpq_status st = cpq::check_dtype("affine_qmm_n", dtype);
  if (st != CPQ_OK) return st;
  st = cpq_quantization_validate(bits, group_size);
  if (st != CPQ_OK) return st;
  if (n % group_size != 0 || n % 32 != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: N=" + std::to_string(n) +
                                              " must be a multiple of 32 and of group_size=" +
                                              std::to_string(group_size));
  if (k % 8 != 0) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: K=" + std::to_string(k) + " must be a multiple of 8");
  size_t kn, mk, mn;
  if (!cpq::mul_ok(k, n, &kn) || !cpq::mul_ok(m, k, &mk) || !cpq::mul_ok(m, n, &mn))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: sizes overflow usize");
  if (w_q_len != kn / 32 * bits)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: w_q.len()=" + std::to_string(w_q_len) + " != K*N*bits/32 (" +
                                              std::to_string(kn / 32 * bits) + ")");
  if (scales_len != kn / group_size || biases_len != kn / group_size)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: scales/biases length mismatch (expected " +
                                              std::to_string(kn / group_size) + ")");
  if (x_len != mk) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: x.len() != M*K");
  if (y_len != mn) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: y.len() != M*N");
  if (m > 0x7fffffff || n > 0x7fffffff || k > 0x7fffffff)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: dimensions beyond 32-bit indexing");
  if (!cpq::kernel_available(dtype, group_size, bits)) return cpq::not_found("qmm_n", dtype, group_size, bits);
  return CPQ_OK;
}

// ---------------------------------------------------------------------------
// Ops
// ---------------------------------------------------------------------------

cpq_status cpq_affine_qmv(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                          size_t w_q_len, const void* scales, size_t scales_len,
                          const void* biases, size_t biases_len, const void* x,
                          size_t x_alloc_bytes, void* y, size_t y_len, size_t in_vec_size,
                          uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv: NULL command session");
  cpq_status st = cpq_check_qmv_args(dtype, w_q_len, scales_len, biases_len, x_alloc_bytes, y_len,
                                     in_vec_size, group_size, bits);
  if (st != CPQ_OK) return st;
  st = cpq::check_ptrs("affine_qmv", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  return cpq::launched(cpq::launch_qmv(cmds->stream, q, x, y, (int)y_len, (int)in_vec_size),
                       "affine_qmv launch");
}

cpq_status cpq_affine_qmm_t(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                            size_t w_q_len, const void* scales, size_t scales_len,
                            const void* biases, size_t biases_len, const void* x, size_t x_len,
                            void* y, size_t y_len, size_t m, size_t n, size_t k,
                            uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t: NULL command session");
  cpq_status st = cpq_check_qmm_args(dtype, w_q_len, scales_len, biases_len, x_len, y_len, m, n, k,
                                     group_size, bits);
  if (st != CPQ_OK) return st;
  st = cpq::check_ptrs("affine_qmm_t", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  // The kernel is chosen by M as for the runtime node (small-M kernels, else
  // the prefill plan): a caller of the op gets the same speed at a given
  // shape whichever entry point it uses.
  return cpq::route_matmul(cmds, q, x, y, (int)m, (int)n, (int)k, "affine_qmm_t");
}

// ---------------------------------------------------------------------------
// Batched forms (MLX's `batched` kernels, adjust_matrix_offsets in
// quantized.h:1351-1388): batch element z picks its x, w, scales and biases
// through per-dimension element strides over the batch shape (stride 0
// broadcasts); y is contiguous, one [M, N] block per element.
// ---------------------------------------------------------------------------

namespace {

using cpq::kMaxBatchDims;

int64_t batch_offset(size_t z, int nd, const int* shape, const int64_t* st) {
  int64_t off = 0;
  for (int d = nd - 1; d >= 0; --d) {
    off += (int64_t)(z % (size_t)shape[d]) * st[d];
    z /= (size_t)shape[d];
  }
  return off;
}

// Element count of the batch, and every operand's batch elements inside its
// buffer (largest offset + one matrix <= length) with offsets that keep the
// kernels' alignment (`align` elements).
cpq_status check_batch(const char* op, int nd, const int* shape, const int64_t* const st[4], const size_t extent[4],
                       const size_t len[4], const size_t align[4], size_t* count) {
  const char* names[4] = {"w_q", "scales", "biases", "x"};
  if (nd < 0 || nd > kMaxBatchDims)
    return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": batch_ndims outside 0..=8");
  if (nd && !shape) return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": NULL batch_shape");
  size_t c = 1;
  for (int d = 0; d < nd; ++d) {
    if (shape[d] < 0) return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": negative batch dimension");
    if (!cpq::mul_ok(c, (size_t)shape[d], &c))
      return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": batch size overflows");
  }
  *count = c;
  if (c == 0) return CPQ_OK;
  for (int o = 0; o < 4; ++o) {
    if (nd && !st[o]) return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": NULL " + names[o] + " strides");
    int64_t mx = 0;
    for (int d = 0; d < nd; ++d) {
      if (st[o][d] < 0) return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": negative " + names[o] + " stride");
      if (st[o][d] % (int64_t)align[o] != 0)
        return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": " + names[o] + " stride " +
                                                  std::to_string(st[o][d]) + " breaks its " +
                                                  std::to_string(align[o]) + "-element alignment");
      if (shape[d] > 1 && st[o][d] > (INT64_MAX - mx) / (shape[d] - 1))
        return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": batch offsets overflow");
      mx += (int64_t)(shape[d] - 1) * st[o][d];
    }
    if ((uint64_t)mx + extent[o] > len[o])
      return fail(CPQ_ERR_INVALID_ARGUMENT, std::string(op) + ": " + names[o] + " batch elements reach past its " +
                                                std::to_string(len[o]) + " elements");
  }
  return CPQ_OK;
}

// No weight operand (w_q, scales, biases) moves along the batch.
bool weights_shared(int nd, const int* shape, const int64_t* const st[4]) {
  for (int d = 0; d < nd; ++d)
    if (shape[d] > 1 && (st[0][d] || st[1][d] || st[2][d])) return false;
  return true;
}

// Element z's activations start at z * block: the batch of x is one dense
// row-major array of blocks.
bool x_dense(int nd, const int* shape, const int64_t* xst, size_t block) {
  uint64_t span = block;
  for (int d = nd - 1; d >= 0; --d) {
    if (shape[d] > 1 && (uint64_t)xst[d] != span) return false;
    span *= (uint64_t)shape[d];
  }
  return true;
}

// The batch as kernel arguments; false when an element's scales or biases
// would lose the 8-byte alignment the decode-layout kernels load with, or
// the batch does not fit a grid dimension.
bool batch_args(int nd, const int* shape, const int64_t* const st[4], size_t count, const void* scales,
                const void* biases, cpq::BatchArgs* ba) {
  if (count > 65535) return false;
  if (((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) & 7u) != 0) return false;
  *ba = cpq::BatchArgs{};
  ba->nd = nd;
  for (int d = 0; d < nd; ++d) {
    if (st[1][d] % 4 || st[2][d] % 4) return false;
    ba->shape[d] = shape[d];
    for (int o = 0; o < 4; ++o) ba->st[o][d] = st[o][d];
  }
  return true;
}

}  // namespace

cpq_status cpq_affine_qmm_t_batched(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                                    const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                                    const void* x, size_t x_len, void* y, size_t y_len, size_t m, size_t n,
                                    size_t k, uint32_t group_size, uint32_t bits, int batch_ndims,
                                    const int* batch_shape, const int64_t* w_strides, const int64_t* s_strides,
                                    const int64_t* b_strides, const int64_t* x_strides) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t_batched: NULL command session");
  size_t mk, mn, nk;
  if (!cpq::mul_ok(m, k, &mk) || !cpq::mul_ok(m, n, &mn) || !cpq::mul_ok(n, k, &nk))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t_batched: sizes overflow usize");
  const size_t words = nk / 32 * bits, groups = group_size ? nk / group_size : 0;
  cpq_status st = cpq_check_qmm_args(dtype, words, groups, groups, mk, mn, m, n, k, group_size, bits);
  if (st != CPQ_OK) return st;
  const int64_t* strides[4] = {w_strides, s_strides, b_strides, x_strides};
  const size_t extent[4] = {words, groups, groups, mk};
  const size_t len[4] = {w_q_len, scales_len, biases_len, x_len};
  const size_t align[4] = {4, 1, 1, 8};  // 16-byte weight and activation rows
  size_t count;
  st = check_batch("affine_qmm_t_batched", batch_ndims, batch_shape, strides, extent, len, align, &count);
  if (st != CPQ_OK) return st;
  size_t ylen;
  if (!cpq::mul_ok(count, mn, &ylen) || y_len != ylen)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t_batched: y.len() != batch*M*N");
  if (count == 0 || mn == 0) return CPQ_OK;
  const size_t esz = cpq::dtype_size(dtype);
  st = cpq::check_ptrs("affine_qmm_t_batched", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  const cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  if (count > 1 && weights_shared(batch_ndims, batch_shape, strides) &&
      x_dense(batch_ndims, batch_shape, x_strides, mk) && count * m <= (size_t)INT32_MAX) {
    // One weight for every element and the activations one dense array:
    // a single matmul over count * M rows (the weights are read once).
    return cpq::route_matmul(cmds, q, x, y, (int)(count * m), (int)n, (int)k, "affine_qmm_t_batched");
  }
  cpq::BatchArgs ba;
  if (count > 1 && m <= 16 && cpq::qmv_rows_fits(q, (int)m, (int)n, (int)k, x) &&
      batch_args(batch_ndims, batch_shape, strides, count, scales, biases, &ba)) {
    // Few rows per element: the decode layout with the batch in its grid.
    return cpq::launched(cpq::launch_qmv_rows_batched(cmds->stream, q, x, y, (int)m, (int)n, (int)k, (int)count, ba),
                         "affine_qmm_t_batched launch");
  }
  for (size_t z = 0; z < count; ++z) {
    const uint32_t* wz = w_q + batch_offset(z, batch_ndims, batch_shape, w_strides);
    const char* sz = static_cast<const char*>(scales) + batch_offset(z, batch_ndims, batch_shape, s_strides) * esz;
    const char* bz = static_cast<const char*>(biases) + batch_offset(z, batch_ndims, batch_shape, b_strides) * esz;
    const char* xz = static_cast<const char*>(x) + batch_offset(z, batch_ndims, batch_shape, x_strides) * esz;
    char* yz = static_cast<char*>(y) + z * mn * esz;
    st = cpq_affine_qmm_t(cmds, dtype, wz, words, sz, groups, bz, groups, xz, mk, yz, mn, m, n, k, group_size, bits);
    if (st != CPQ_OK) return st;
  }
  return CPQ_OK;
}

cpq_status cpq_affine_qmv_batched(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                                  const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                                  const void* x, size_t x_len, void* y, size_t y_len, size_t n, size_t k,
                                  uint32_t group_size, uint32_t bits, int batch_ndims, const int* batch_shape,
                                  const int64_t* w_strides, const int64_t* s_strides, const int64_t* b_strides,
                                  const int64_t* x_strides) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv_batched: NULL command session");
  size_t nk;
  if (!cpq::mul_ok(n, k, &nk)) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv_batched: N*K overflows usize");
  const size_t words = nk / 32 * bits, groups = group_size ? nk / group_size : 0;
  const size_t esz = cpq::dtype_size(dtype);
  cpq_status st = cpq_check_qmv_args(dtype, words, groups, groups, k * esz, n, k, group_size, bits);
  if (st != CPQ_OK) return st;
  const int64_t* strides[4] = {w_strides, s_strides, b_strides, x_strides};
  const size_t extent[4] = {words, groups, groups, k};
  const size_t len[4] = {w_q_len, scales_len, biases_len, x_len};
  const size_t align[4] = {4, 1, 1, 8};
  size_t count;
  st = check_batch("affine_qmv_batched", batch_ndims, batch_shape, strides, extent, len, align, &count);
  if (st != CPQ_OK) return st;
  size_t ylen;
  if (!cpq::mul_ok(count, n, &ylen) || y_len != ylen)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmv_batched: y.len() != batch*N");
  if (count == 0 || n == 0) return CPQ_OK;
  st = cpq::check_ptrs("affine_qmv_batched", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  const cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  if (count > 1 && n % 32 == 0 && weights_shared(batch_ndims, batch_shape, strides) &&
      x_dense(batch_ndims, batch_shape, x_strides, k) && count <= (size_t)INT32_MAX) {
    // One weight for every element and the activations one dense array:
    // a single matmul over count rows (the weights are read once).
    return cpq::route_matmul(cmds, q, x, y, (int)count, (int)n, (int)k, "affine_qmv_batched");
  }
  cpq::BatchArgs ba;
  if (count > 1 && cpq::qmv_batch_fits(q, (int)n, (int)k) &&
      batch_args(batch_ndims, batch_shape, strides, count, scales, biases, &ba)) {
    // The decode kernel with the batch in its grid.
    return cpq::launched(cpq::launch_qmv_batched(cmds->stream, q, x, y, (int)n, (int)k, (int)count, ba),
                         "affine_qmv_batched launch");
  }
  for (size_t z = 0; z < count; ++z) {
    const uint32_t* wz = w_q + batch_offset(z, batch_ndims, batch_shape, w_strides);
    const char* sz = static_cast<const char*>(scales) + batch_offset(z, batch_ndims, batch_shape, s_strides) * esz;
    const char* bz = static_cast<const char*>(biases) + batch_offset(z, batch_ndims, batch_shape, b_strides) * esz;
    const char* xz = static_cast<const char*>(x) + batch_offset(z, batch_ndims, batch_shape, x_strides) * esz;
    char* yz = static_cast<char*>(y) + z * n * esz;
    st = cpq_affine_qmv(cmds, dtype, wz, words, sz, groups, bz, groups, xz, k * esz, yz, n, k, group_size, bits);
    if (st != CPQ_OK) return st;
  }
  return CPQ_OK;
}

cpq_status cpq_affine_dequantize(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                                 size_t w_q_len, const void* scales, size_t scales_len,
                                 const void* biases, size_t biases_len, void* out,
                                 size_t out_len, uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_dequantize: NULL command session");
  cpq_status st = cpq_check_dequantize_args(dtype, w_q_len, scales_len, biases_len, out_len,
                                            group_size, bits);
  if (st != CPQ_OK) return st;
  if (out_len == 0) return CPQ_OK;
  st = cpq::check_ptrs("affine_dequantize", w_q, scales, biases, out, out);
  if (st != CPQ_OK) return st;
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  return cpq::launched(cpq::launch_dequantize(cmds->stream, q, out, out_len),
                       "affine_dequantize launch");
}

cpq_status cpq_affine_qmm_n(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                            const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                            const void* x, size_t x_len, void* y, size_t y_len, size_t m, size_t n, size_t k,
                            uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_n: NULL command session");
  cpq_status st = cpq_check_qmm_n_args(dtype, w_q_len, scales_len, biases_len, x_len, y_len, m, n, k, group_size,
                                       bits);
  if (st != CPQ_OK) return st;
  if (m == 0 || n == 0) return CPQ_OK;
  st = cpq::check_ptrs("affine_qmm_n", k ? w_q : reinterpret_cast<const uint32_t*>(y), k ? scales : y,
                       k ? biases : y, k ? x : y, y);
  if (st != CPQ_OK) return st;
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  if (m == 1 && k > 0 && (reinterpret_cast<uintptr_t>(x) & 3u) == 0 && cpq::qvm_fits(q, (int)n, (int)k)) {
    // Decode (qvm): the VALU kernel, K split over parts that meet in the
    // session scratch when it holds them (the plan depends on the session's
    // fixed capacity only).
    const cpq::QvmPlan plan = cpq::qvm_plan(q, (int)n, (int)k, cmds->dev ? cmds->dev->cu_count : 0,
                                            cmds->scratch ? cmds->scratch_bytes : 0);
    void* scratch = nullptr;
    if (plan.scratch_bytes) cpq::session_scratch(cmds, plan.scratch_bytes, &scratch);
    return cpq::launched(cpq::launch_qvm(cmds->stream, plan, scratch, q, x, y, (int)n, (int)k), "affine_qvm launch");
  }
  // Few output tiles: split K into fp32 partials in session scratch (past the
  // prefill kernel's counters) when the session's scratch holds them, else
  // no split (the choice depends on the shape and the session only).
  int split = cpq::qmm_n_split((int)m, (int)n, (int)k, cmds->dev ? cmds->dev->cu_count : 0);
  float* partial = nullptr;
  if (split > 1) {
    void* scratch = nullptr;
    if (cpq::session_scratch(cmds, cpq::kWideCounterBytes + cpq::qmm_n_scratch_bytes((int)m, (int)n, split),
                             &scratch))
      partial = reinterpret_cast<float*>(static_cast<char*>(scratch) + cpq::kWideCounterBytes);
    else
      split = 1;
  }
  return cpq::launched(cpq::launch_qmm_n(cmds->stream, q, x, y, (int)m, (int)n, (int)k, split, partial),
                       "affine_qmm_n launch");
}

cpq_status cpq_embed_tokens(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q, size_t w_q_len,
                            const void* scales, size_t scales_len, const void* biases, size_t biases_len,
                            const uint32_t* ids, size_t n_ids, size_t vocab, size_t hidden, void* out,
                            size_t out_len, uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: NULL command session");
  cpq_status st = cpq_check_embed_args(dtype, w_q_len, scales_len, biases_len, n_ids, vocab, hidden, out_len,
                                       group_size, bits);
  if (st != CPQ_OK) return st;
  if (n_ids == 0) return CPQ_OK;
  st = cpq::check_ptrs("embed_tokens", w_q, scales, biases, out, out);
  if (st != CPQ_OK) return st;
  if (!ids || (reinterpret_cast<uintptr_t>(ids) & 3u))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "embed_tokens: ids must be a non-NULL, 4-byte aligned device pointer");
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  return cpq::launched(cpq::launch_embed(cmds->stream, q, ids, (uint32_t)n_ids, (uint32_t)vocab, (uint32_t)hidden,
                                         out, cmds->status + 1),
                       "embed_tokens launch");
}

// Routed-expert plumbing (no reference counterpart: feed-forward.md:98-107
// names the router, top-k and gather_qmm feed as unbuilt).
cpq_status cpq_moe_route(cpq_commands* cmds, cpq_dtype logits_dtype, const void* logits, size_t tokens,
                         size_t n_experts, uint32_t top_k, int normalize, uint32_t* experts, float* scores,
                         uint32_t* lhs, uint32_t* rhs, uint32_t* inv, uint32_t* offsets) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: NULL command session");
  cpq_status st = cpq::check_dtype("moe_route", logits_dtype);
  if (st != CPQ_OK) return st;
  if (n_experts == 0 || n_experts > 1024)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: n_experts=" + std::to_string(n_experts) + " outside 1..=1024");
  if (top_k == 0 || top_k > 16 || top_k > n_experts)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: top_k=" + std::to_string(top_k) +
                                              " outside 1..=min(16, n_experts)");
  size_t rows;
  if (!cpq::mul_ok(tokens, top_k, &rows) || rows >= (1ull << 31) || tokens * n_experts / n_experts != tokens)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: tokens*top_k beyond 32-bit indexing");
  if (!offsets) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: NULL offsets");
  if (tokens && (!logits || !experts || !scores || !lhs || !rhs || !inv))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_route: NULL buffer");
  void* scratch = nullptr;
  const size_t need = cpq::kWideCounterBytes + cpq::moe_sort_scratch_bytes((int)rows, (int)n_experts);
  if (!cpq::session_scratch(cmds, need, &scratch))
    return fail(CPQ_ERR_BUFFER_TOO_LARGE, "moe_route: the sort needs " + std::to_string(need) +
                                              " bytes of session scratch; the session holds " +
                                              std::to_string(cmds->scratch_bytes) +
                                              " (CPQ_SESSION_SCRATCH_MB sets it when the session is made)");
  // The scratch head holds the prefill kernel's arrival counters; the sort's
  // block histograms go after it.
  uint32_t* hist = reinterpret_cast<uint32_t*>(static_cast<char*>(scratch) + cpq::kWideCounterBytes);
  st = cpq::launched(cpq::launch_moe_route(cmds->stream, (int)logits_dtype, logits, (int)tokens, (int)n_experts,
                                           (int)top_k, normalize, experts, scores),
                     "moe_route launch");
  if (st != CPQ_OK) return st;
  return cpq::launched(cpq::launch_moe_sort(cmds->stream, experts, (int)rows, (int)top_k, (int)n_experts, hist, lhs,
                                            rhs, inv, offsets),
                       "moe_route sort launch");
}

cpq_status cpq_moe_combine(cpq_commands* cmds, cpq_dtype dtype, const void* y, size_t y_len, const float* scores,
                           const uint32_t* inv, size_t tokens, uint32_t top_k, size_t n, void* out, size_t out_len) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: NULL command session");
  if (dtype != CPQ_DTYPE_BF16 && dtype != CPQ_DTYPE_F16)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: dtype must be BF16 or F16");
  if (top_k == 0 || top_k > 16) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: top_k outside 1..=16");
  if (n % 8 != 0) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: N must be a multiple of 8");
  size_t rows, yl, ol;
  if (!cpq::mul_ok(tokens, top_k, &rows) || rows >= (1ull << 31) || !cpq::mul_ok(rows, n, &yl) ||
      !cpq::mul_ok(tokens, n, &ol))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: sizes overflow");
  if (y_len != yl) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: y.len() != tokens*top_k*N");
  if (out_len != ol) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: out.len() != tokens*N");
  if (tokens == 0 || n == 0) return CPQ_OK;
  if (!y || !scores || !inv || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: NULL buffer");
  if ((reinterpret_cast<uintptr_t>(y) | reinterpret_cast<uintptr_t>(out)) & 15u)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "moe_combine: y and out must be 16-byte aligned");
  return cpq::launched(cpq::launch_moe_combine(cmds->stream, (int)dtype, y, scores, inv, (int)tokens, (int)top_k,
                                               (int)n, out, cmds->status + 2),
                       "moe_combine launch");
}

cpq_status cpq_affine_gather_qmm(cpq_commands* cmds, cpq_dtype dtype, const void* x,
                                 size_t x_rows, const uint32_t* w_q, size_t w_q_len,
                                 const void* scales, size_t scales_len, const void* biases,
                                 size_t biases_len, const uint32_t* lhs_indices,
                                 const uint32_t* rhs_indices, size_t n_rows, void* y,
                                 size_t y_len, size_t n_experts, size_t n, size_t k,
                                 uint32_t group_size, uint32_t bits, int sorted_indices) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: NULL command session");
  cpq_status st = cpq_check_gather_args(dtype, x_rows, w_q_len, scales_len, biases_len,
                                        lhs_indices != nullptr, n_rows, y_len, n_experts, n, k,
                                        group_size, bits);
  if (st != CPQ_OK) return st;
  if (n_rows == 0) return CPQ_OK;
  if (!rhs_indices) return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: rhs_indices is NULL");
  st = cpq::check_ptrs("affine_gather_qmm", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  if (x_rows == 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_gather_qmm: x has no rows but lhs_indices select some");
  if (!cpq::gather_supported((int)bits, (int)n_rows, (int)n, (int)k, (int)group_size))
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_gather_qmm: K=" + std::to_string(k) + " at group_size " + std::to_string(group_size) +
                    " has " + std::to_string(k / group_size) +
                    " groups per row: beyond what the per-slab routed kernel holds in LDS (about 600), and "
                    "outside the expert-major kernel's shapes (4- or 8-bit, K % 128 == 0, bounded K and rows)");
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  return cpq::launched(cpq::launch_gather_qmm(cmds->stream, q, x, (int)x_rows, lhs_indices,
                                              rhs_indices, (int)n_rows, y, (int)n_experts, (int)n,
                                              (int)k, sorted_indices != 0, cmds->status),
                       "affine_gather_qmm launch");
}

cpq_status cpq_stream_read_variant(cpq_commands* cmds, const void* const* regions, const size_t* bytes,
                                   int n_regions, uint32_t* sink, int n_workgroups, int variant) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: NULL command session");
  if (n_regions < 1 || n_regions > 4 || !regions || !bytes)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: 1..=4 regions with their lengths");
  if (n_workgroups < 1 || n_workgroups > 65535)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: n_workgroups outside 1..=65535");
  if (variant < 0 || variant >= cpq::stream_read_variant_count())
    return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: variant outside 0..=" +
                                              std::to_string(cpq::stream_read_variant_count() - 1));
  if (!sink || (reinterpret_cast<uintptr_t>(sink) & 3u))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: sink must be a 4-byte aligned device pointer");
  uint64_t total = 0;
  for (int g = 0; g < n_regions; ++g) {
    if ((bytes[g] && !regions[g]) || !cpq::aligned16(regions[g]) || bytes[g] % 16 != 0)
      return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: region " + std::to_string(g) +
                                                " must be 16-byte aligned with a length that is a multiple of 16");
    total += bytes[g];
  }
  // The buffer-addressed designs cover one workgroup's span with a 32-bit
  // byte range.
  if (total / (uint64_t)n_workgroups + 16 >= (1ull << 32))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "stream_read: more than 4 GiB per workgroup");
  return cpq::launched(cpq::launch_stream_read(cmds->stream, regions, bytes, n_regions, sink, n_workgroups, variant),
                       "stream_read launch");
}

cpq_status cpq_stream_read(cpq_commands* cmds, const void* const* regions, const size_t* bytes, int n_regions,
                           uint32_t* sink, int n_workgroups) {
  return cpq_stream_read_variant(cmds, regions, bytes, n_regions, sink, n_workgroups, 0);
}

int cpq_stream_read_variant_count(void) { return cpq::stream_read_variant_count(); }

cpq_status cpq_quantized_matmul(cpq_commands* cmds, cpq_dtype dtype, const uint32_t* w_q,
                                size_t w_q_len, const void* scales, size_t scales_len,
                                const void* biases, size_t biases_len, const void* x, size_t x_len,
                                size_t x_alloc_bytes, void* y, size_t m, size_t n,
                                size_t k_physical, uint32_t group_size, uint32_t bits) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: NULL command session");
  if (m == 0) return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: activation has no rows");
  if (m == 1) {
    // eval.rs:1360-1372: M == 1 -> qmv (K-padded activations allowed).
    return cpq_affine_qmv(cmds, dtype, w_q, w_q_len, scales, scales_len, biases, biases_len, x,
                          x_alloc_bytes, y, n, k_physical, group_size, bits);
  }
  // eval.rs:1377-1390: M > 1 -> qmm_t contract (x.len() == M*K, N % 32 == 0);
  // a K-padded weight self-rejects here because x_len == M*k_logical.
  if (x_alloc_bytes < x_len * cpq::dtype_size(dtype))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: x allocation smaller than x_len");
  size_t mn;
  if (!cpq::mul_ok(m, n, &mn)) return fail(CPQ_ERR_INVALID_ARGUMENT, "quantized_matmul: M*N overflows usize");
  cpq_status st = cpq_check_qmm_args(dtype, w_q_len, scales_len, biases_len, x_len, mn, m, n,
                                     k_physical, group_size, bits);
  if (st != CPQ_OK) return st;
  st = cpq::check_ptrs("quantized_matmul", w_q, scales, biases, x, y);
  if (st != CPQ_OK) return st;
  cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  return cpq::route_matmul(cmds, q, x, y, (int)m, (int)n, (int)k_physical, "quantized_matmul");
}

}  // extern "C"
