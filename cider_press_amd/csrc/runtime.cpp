// Device, buffer, command-session, event and error plumbing of libcpq.so.
//
// Replaces the reference's Metal dispatch/buffer layer
// (crates/cider-press-kernels/src/{device,buffer,commands,error}.rs) with HIP:
// one in-order hipStream per command session instead of an MTLCommandBuffer,
// hipMalloc'd device memory instead of shared MTLBuffers.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "cpq_internal.hpp"

namespace {
thread_local std::string g_last_error;
constexpr size_t kAllocGranule = 512;  // device.rs:191-224 rounds every allocation to 512 B
}  // namespace

namespace cpq {

cpq_status fail(cpq_status st, const std::string& msg) {
  g_last_error = msg;
  return st;
}

cpq_status hip_fail(hipError_t e, const char* what) {
  std::string m = std::string(what) + ": " + hipGetErrorName(e) + " (" + hipGetErrorString(e) + ")";
  g_last_error = m;
  return CPQ_ERR_HIP_API;
}

bool session_scratch(const cpq_commands* c, size_t bytes, void** out) {
  if (!c->scratch || bytes > c->scratch_bytes) return false;
  *out = c->scratch;
  return true;
}

}  // namespace cpq

using cpq::fail;
using cpq::hip_fail;

extern "C" {

const char* cpq_last_error_message(void) { return g_last_error.c_str(); }

const char* cpq_version(void) { return "cpq 0.1.0 (gfx950)"; }

// ---------------------------------------------------------------------------
// Device
// ---------------------------------------------------------------------------

cpq_status cpq_device_system_default(cpq_device** out) {
  if (!out) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_device_system_default: out is NULL");
  *out = nullptr;
  int count = 0;
  hipError_t e = hipGetDeviceCount(&count);
  if (e != hipSuccess || count <= 0)
    return fail(CPQ_ERR_NO_DEVICE, "no HIP device available on this system");
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, 0);
  if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(CPQ_ERR_NO_DEVICE, std::string("device 0 is ") + prop.gcnArchName +
                                       "; libcpq is built for gfx950 only");
  e = hipSetDevice(0);
  if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
  auto* d = new cpq_device();
  d->ordinal = 0;
  d->cu_count = prop.multiProcessorCount;
  d->clock_khz = prop.clockRate;
  if (prop.name[0])
    std::snprintf(d->name, sizeof(d->name), "%s (%s)", prop.name, prop.gcnArchName);
  else  // the marketing name is not always readable on shared boxes
    std::snprintf(d->name, sizeof(d->name), "%s, %d CUs", prop.gcnArchName, prop.multiProcessorCount);
  *out = d;
  return CPQ_OK;
}

void cpq_device_release(cpq_device* dev) {
  if (!dev) return;
  if (dev->eval_session) cpq_commands_release(dev->eval_session);
  delete dev;
}

cpq_status cpq_device_info(cpq_device* dev, char* name, size_t name_cap, int* cu_count,
                           int* clock_khz) {
  if (!dev) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_device_info: device is NULL");
  if (name && name_cap) {
    std::strncpy(name, dev->name, name_cap - 1);
    name[name_cap - 1] = 0;
  }
  if (cu_count) *cu_count = dev->cu_count;
  if (clock_khz) *clock_khz = dev->clock_khz;
  return CPQ_OK;
}

// ---------------------------------------------------------------------------
// Buffers
// ---------------------------------------------------------------------------

cpq_status cpq_alloc_buffer(cpq_device* dev, size_t byte_len, void** out_ptr,
                            size_t* out_alloc_len) {
  if (!dev || !out_ptr) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_alloc_buffer: NULL argument");
  *out_ptr = nullptr;
  if (byte_len > SIZE_MAX - kAllocGranule)
    return fail(CPQ_ERR_BUFFER_TOO_LARGE,
                "buffer length " + std::to_string(byte_len) + " bytes overflows the 512-B rounding");
  // A zero-length buffer still owns one granule so a device pointer exists.
  size_t alloc = byte_len == 0 ? kAllocGranule
                               : (byte_len + kAllocGranule - 1) / kAllocGranule * kAllocGranule;
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, alloc);
  if (e != hipSuccess || !p)
    return fail(CPQ_ERR_BUFFER_ALLOCATION,
                "failed to allocate device buffer of " + std::to_string(alloc) + " bytes");
  // Zero the slack [byte_len, alloc): a K-padded read past the logical end
  // must see 0.0, never a stale NaN (qmv.rs:95-116).
  if (alloc > byte_len) {
    e = hipMemset(static_cast<char*>(p) + byte_len, 0, alloc - byte_len);
    if (e != hipSuccess) {
      (void)hipFree(p);
      return hip_fail(e, "hipMemset(slack)");
    }
  }
  *out_ptr = p;
  if (out_alloc_len) *out_alloc_len = alloc;
  return CPQ_OK;
}

cpq_status cpq_upload(cpq_device* dev, const void* host, size_t byte_len, void** out_ptr,
                      size_t* out_alloc_len) {
  if (byte_len && !host) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_upload: host is NULL");
  cpq_status st = cpq_alloc_buffer(dev, byte_len, out_ptr, out_alloc_len);
  if (st != CPQ_OK) return st;
  if (byte_len) {
    hipError_t e = hipMemcpy(*out_ptr, host, byte_len, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
      (void)hipFree(*out_ptr);
      *out_ptr = nullptr;
      return hip_fail(e, "hipMemcpy(upload)");
    }
  }
  return CPQ_OK;
}

cpq_status cpq_free_buffer(cpq_device* dev, void* ptr) {
  (void)dev;
  if (!ptr) return CPQ_OK;
  hipError_t e = hipFree(ptr);
  if (e != hipSuccess) return hip_fail(e, "hipFree");
  return CPQ_OK;
}

cpq_status cpq_read_buffer(cpq_device* dev, const void* dev_ptr, void* host, size_t byte_len) {
  (void)dev;
  if (!byte_len) return CPQ_OK;
  if (!dev_ptr || !host) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_read_buffer: NULL pointer");
  hipError_t e = hipMemcpy(host, dev_ptr, byte_len, hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy(read)");
  return CPQ_OK;
}

cpq_status cpq_write_buffer(cpq_device* dev, void* dev_ptr, const void* host, size_t byte_len) {
  (void)dev;
  if (!byte_len) return CPQ_OK;
  if (!dev_ptr || !host) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_write_buffer: NULL pointer");
  hipError_t e = hipMemcpy(dev_ptr, host, byte_len, hipMemcpyHostToDevice);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy(write)");
  return CPQ_OK;
}

// ---------------------------------------------------------------------------
// Command sessions
// ---------------------------------------------------------------------------

static cpq_status make_commands(cpq_device* dev, hipStream_t stream, bool owns,
                                cpq_commands** out) {
  unsigned int* status = nullptr;
  hipError_t e = hipMalloc(&status, 3 * sizeof(unsigned int));
  if (e != hipSuccess) return hip_fail(e, "hipMalloc(status word)");
  e = hipMemset(status, 0, 3 * sizeof(unsigned int));
  if (e != hipSuccess) {
    (void)hipFree(status);
    return hip_fail(e, "hipMemset(status word)");
  }
  auto* c = new cpq_commands();
  c->dev = dev;
  c->stream = stream;
  c->owns_stream = owns;
  c->status = status;
  // Scratch of the session's split-K reductions and routing sort, allocated
  // here once with a fixed capacity (CPQ_SESSION_SCRATCH_MB, default 64 MiB:
  // the arrival counters plus 1023 fp32 partial tiles of 128 x 128).  Ops
  // never grow it, so the kernel an op selects depends on the shape and this
  // capacity only -- never on whether the stream is being captured into a
  // graph.  Without it (0, or the allocation failed) split-K kernels are not
  // selected.
  const char* env = std::getenv("CPQ_SESSION_SCRATCH_MB");
  const long mb = env && *env ? std::atol(env) : (long)(cpq::kDefaultSessionScratchBytes >> 20);
  if (mb > 0) {
    void* p = nullptr;
    if (hipMalloc(&p, (size_t)mb << 20) == hipSuccess) {
      // Counters start at zero; a kernel (not a memset) keeps the stream free
      // of memset nodes should it be captured later.
      if (cpq::zero_words(stream, p, cpq::kWideCounterBytes / 4) == hipSuccess &&
          hipStreamSynchronize(stream) == hipSuccess) {
        c->scratch = p;
        c->scratch_bytes = (size_t)mb << 20;
      } else {
        (void)hipFree(p);
      }
    }
    (void)hipGetLastError();
  }
  *out = c;
  return CPQ_OK;
}

cpq_status cpq_commands_create(cpq_device* dev, cpq_commands** out) {
  if (!dev || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_commands_create: NULL argument");
  *out = nullptr;
  hipStream_t s = nullptr;
  // Default priority on purpose: no stream-priority games.
  hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
  if (e != hipSuccess) return hip_fail(e, "hipStreamCreateWithFlags");
  cpq_status st = make_commands(dev, s, true, out);
  if (st != CPQ_OK) (void)hipStreamDestroy(s);
  return st;
}

cpq_status cpq_commands_wrap_stream(cpq_device* dev, void* hip_stream, cpq_commands** out) {
  if (!dev || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_commands_wrap_stream: NULL argument");
  *out = nullptr;
  return make_commands(dev, static_cast<hipStream_t>(hip_stream), false, out);
}

void* cpq_commands_stream(cpq_commands* cmds) { return cmds ? cmds->stream : nullptr; }

cpq_status cpq_commands_commit(cpq_commands* cmds) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_commands_commit: NULL session");
  return CPQ_OK;
}

cpq_status cpq_commands_wait(cpq_commands* cmds) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_commands_wait: NULL session");
  hipError_t e = hipStreamSynchronize(cmds->stream);
  if (e != hipSuccess) return cpq_completion_result((int)e);
  unsigned int bad[3] = {0u, 0u, 0u};
  e = hipMemcpy(bad, cmds->status, sizeof(bad), hipMemcpyDeviceToHost);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpy(status word)");
  if (bad[0] || bad[1] || bad[2]) {
    e = hipMemset(cmds->status, 0, sizeof(bad));
    if (e != hipSuccess) return hip_fail(e, "hipMemset(status word)");
    std::string msg;
    if (bad[0])
      msg = "affine_gather_qmm: " + std::to_string(bad[0]) +
            " row(s) carried an out-of-range lhs/rhs index (written as 0) or broke the ascending order "
            "promised by sorted_indices";
    if (bad[1])
      msg += std::string(msg.empty() ? "" : "; ") + "embed_tokens: " + std::to_string(bad[1]) +
             " id(s) at or past the vocabulary size; those rows were written as 0";
    if (bad[2])
      msg += std::string(msg.empty() ? "" : "; ") + "moe_combine: " + std::to_string(bad[2]) +
             " (token, slot) position(s) outside the expert rows; they contributed 0";
    return fail(CPQ_ERR_INVALID_ARGUMENT, msg);
  }
  return CPQ_OK;
}

cpq_status cpq_commands_commit_and_wait(cpq_commands* cmds) {
  cpq_status st = cpq_commands_commit(cmds);
  if (st != CPQ_OK) return st;
  return cpq_commands_wait(cmds);
}

void cpq_commands_release(cpq_commands* cmds) {
  if (!cmds) return;
  if (cmds->stream) (void)hipStreamSynchronize(cmds->stream);
  for (hipEvent_t ev : cmds->prof_events) (void)hipEventDestroy(ev);
  if (cmds->status) (void)hipFree(cmds->status);
  if (cmds->scratch) (void)hipFree(cmds->scratch);
  if (cmds->owns_stream && cmds->stream) (void)hipStreamDestroy(cmds->stream);
  delete cmds;
}

// ---------------------------------------------------------------------------
// Encoder hazard hooks (commands.rs:139-153, 290-296).  One in-order stream
// per session orders every launch after the previous one, so there is no
// fence to wait or barrier to elide; the hooks only check the session.
// ---------------------------------------------------------------------------

cpq_status cpq_commands_record_input(cpq_commands* cmds, uint64_t) {
  return cmds ? CPQ_OK : fail(CPQ_ERR_INVALID_ARGUMENT, "record_input: NULL session");
}

cpq_status cpq_commands_record_output(cpq_commands* cmds, uint64_t) {
  return cmds ? CPQ_OK : fail(CPQ_ERR_INVALID_ARGUMENT, "record_output: NULL session");
}

cpq_status cpq_commands_record_unresolved_input(cpq_commands* cmds) {
  return cmds ? CPQ_OK : fail(CPQ_ERR_INVALID_ARGUMENT, "record_unresolved_input: NULL session");
}

cpq_status cpq_commands_elide_next_barrier(cpq_commands* cmds) {
  return cmds ? CPQ_OK : fail(CPQ_ERR_INVALID_ARGUMENT, "elide_next_barrier: NULL session");
}

// ---------------------------------------------------------------------------
// Profiled sessions: per-op GPU windows from timing events on the session's
// stream (GpuSampler, gpu_sampler.rs:44-162; commands.rs:155-181, 361-374).
// ---------------------------------------------------------------------------

int cpq_device_supports_stage_boundary_sampling(cpq_device* dev) { return dev ? 1 : 0; }

cpq_status cpq_device_gpu_timestamp_period_ns(cpq_device* dev, double* out_ns_per_tick) {
  if (!dev || !out_ns_per_tick)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "gpu_timestamp_period_ns: NULL argument");
  *out_ns_per_tick = 1.0;  // segments are resolved to nanoseconds
  return CPQ_OK;
}

cpq_status cpq_commands_create_profiled(cpq_device* dev, size_t op_capacity, cpq_commands** out) {
  if (!dev || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "commands_profiled: NULL argument");
  *out = nullptr;
  if (op_capacity > SIZE_MAX / 2) return fail(CPQ_ERR_HIP_API, "GpuSampler: op_capacity * 2 overflow");
  cpq_commands* c = nullptr;
  cpq_status st = cpq_commands_create(dev, &c);
  if (st != CPQ_OK) return st;
  c->profiled = true;
  c->prof_events.reserve(2 * op_capacity);
  for (size_t i = 0; i < 2 * op_capacity; ++i) {
    hipEvent_t ev = nullptr;
    hipError_t e = hipEventCreate(&ev);
    if (e != hipSuccess) {
      cpq_commands_release(c);
      return hip_fail(e, "GpuSampler: hipEventCreate");
    }
    c->prof_events.push_back(ev);
  }
  *out = c;
  return CPQ_OK;
}

// Ends the open op's window: its end event follows everything encoded for it.
static cpq_status close_profiled_op(cpq_commands* c) {
  if (!c->prof_open) return CPQ_OK;
  c->prof_open = false;
  hipError_t e = hipEventRecord(c->prof_events[c->prof_ops.back().end], c->stream);
  return e == hipSuccess ? CPQ_OK : hip_fail(e, "begin_profiled_op: hipEventRecord(end)");
}

cpq_status cpq_commands_begin_profiled_op(cpq_commands* cmds, const char* label) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "begin_profiled_op: NULL session");
  if (!cmds->profiled) return CPQ_OK;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(cmds->stream, &cap);
  if (e != hipSuccess) return hip_fail(e, "begin_profiled_op: hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "begin_profiled_op: the session's stream is being captured");
  cpq_status st = close_profiled_op(cmds);
  if (st != CPQ_OK) return st;
  // Reserve a (start, end) pair; past capacity, stop timing further ops
  // rather than failing mid-batch (gpu_sampler.rs reserve, commands.rs:172-180).
  const size_t start = cmds->prof_cursor, end = start + 1;
  if (end >= cmds->prof_events.size()) return CPQ_OK;
  cmds->prof_cursor = end + 1;
  cmds->prof_ops.push_back({label ? std::string(label) : std::string(), start, end});
  e = hipEventRecord(cmds->prof_events[start], cmds->stream);
  if (e != hipSuccess) {
    cmds->prof_ops.pop_back();
    cmds->prof_cursor = start;
    return hip_fail(e, "begin_profiled_op: hipEventRecord(start)");
  }
  cmds->prof_open = true;
  return CPQ_OK;
}

cpq_status cpq_commands_profiled_info(cpq_commands* cmds, size_t* recorded_ops, size_t* sample_capacity) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "profiled_info: NULL session");
  if (recorded_ops) *recorded_ops = cmds->prof_ops.size();
  if (sample_capacity) *sample_capacity = cmds->prof_events.size();
  return CPQ_OK;
}

cpq_status cpq_commands_commit_wait_resolve(cpq_commands* cmds, cpq_gpu_segment* out, size_t cap,
                                            size_t* n_out) {
  if (!cmds || !n_out) return fail(CPQ_ERR_INVALID_ARGUMENT, "commit_wait_resolve: NULL argument");
  *n_out = 0;
  const size_t n = cmds->prof_ops.size();
  if (n > cap || (n && !out))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "commit_wait_resolve: room for " + std::to_string(cap) +
                                              " segments, the batch recorded " + std::to_string(n));
  cpq_status st = close_profiled_op(cmds);
  if (st == CPQ_OK) st = cpq_commands_commit_and_wait(cmds);
  std::vector<cpq_commands::ProfiledOp> ops;
  ops.swap(cmds->prof_ops);  // a new batch starts whatever happens below
  cmds->prof_cursor = 0;
  cmds->prof_open = false;
  if (st != CPQ_OK) return st;
  cmds->prof_resolved_labels.clear();
  for (const auto& op : ops) cmds->prof_resolved_labels.push_back(op.label);
  // Offsets from the first op's start; each window from its own event pair,
  // so a window's length keeps full precision however late in the batch.
  for (size_t i = 0; i < n; ++i) {
    float off_ms = 0.0f, len_ms = 0.0f;
    hipError_t e = hipEventElapsedTime(&off_ms, cmds->prof_events[ops[0].start], cmds->prof_events[ops[i].start]);
    if (e == hipSuccess) e = hipEventElapsedTime(&len_ms, cmds->prof_events[ops[i].start], cmds->prof_events[ops[i].end]);
    if (e != hipSuccess) return hip_fail(e, "GpuSampler::resolve: hipEventElapsedTime");
    const uint64_t s = (uint64_t)(std::max(0.0, (double)off_ms * 1e6) + 0.5);
    const uint64_t d = (uint64_t)(std::max(0.0, (double)len_ms * 1e6) + 0.5);
    out[i] = cpq_gpu_segment{cmds->prof_resolved_labels[i].c_str(), s, s + d};
  }
  *n_out = n;
  return CPQ_OK;
}

cpq_status cpq_completion_result(int hip_error) {
  const hipError_t e = static_cast<hipError_t>(hip_error);
  if (e == hipSuccess) return CPQ_OK;
  return fail(CPQ_ERR_COMMAND_BUFFER_FAILED, std::string("GPU command stream failed: ") + hipGetErrorName(e) +
                                                 " (" + hipGetErrorString(e) + ")");
}

// ---------------------------------------------------------------------------
// Graph capture
// ---------------------------------------------------------------------------

cpq_status cpq_commands_begin_capture(cpq_commands* cmds) {
  if (!cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "begin_capture: NULL session");
  hipError_t e = hipStreamBeginCapture(cmds->stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
  return CPQ_OK;
}

cpq_status cpq_commands_end_capture(cpq_commands* cmds, cpq_graph** out) {
  if (!cmds || !out) return fail(CPQ_ERR_INVALID_ARGUMENT, "end_capture: NULL argument");
  *out = nullptr;
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture(cmds->stream, &g);
  if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(e, "hipGraphInstantiate");
  }
  auto* gr = new cpq_graph();
  gr->graph = g;
  gr->exec = x;
  *out = gr;
  return CPQ_OK;
}

cpq_status cpq_graph_launch(cpq_graph* graph, cpq_commands* cmds) {
  if (!graph || !cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "graph_launch: NULL argument");
  hipError_t e = hipGraphLaunch(graph->exec, cmds->stream);
  if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
  return CPQ_OK;
}

void cpq_graph_release(cpq_graph* graph) {
  if (!graph) return;
  if (graph->exec) (void)hipGraphExecDestroy(graph->exec);
  if (graph->graph) (void)hipGraphDestroy(graph->graph);
  delete graph;
}

// ---------------------------------------------------------------------------
// Events
// ---------------------------------------------------------------------------

cpq_status cpq_event_create(cpq_event** out) {
  if (!out) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_event_create: out is NULL");
  auto* ev = new cpq_event();
  hipError_t e = hipEventCreate(&ev->ev);
  if (e != hipSuccess) {
    delete ev;
    *out = nullptr;
    return hip_fail(e, "hipEventCreate");
  }
  *out = ev;
  return CPQ_OK;
}

cpq_status cpq_event_record(cpq_event* ev, cpq_commands* cmds) {
  if (!ev || !cmds) return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_event_record: NULL argument");
  hipError_t e = hipEventRecord(ev->ev, cmds->stream);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  return CPQ_OK;
}

cpq_status cpq_event_elapsed_ms(cpq_event* start, cpq_event* end, float* out_ms) {
  if (!start || !end || !out_ms)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "cpq_event_elapsed_ms: NULL argument");
  hipError_t e = hipEventSynchronize(end->ev);
  if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
  e = hipEventElapsedTime(out_ms, start->ev, end->ev);
  if (e != hipSuccess) return hip_fail(e, "hipEventElapsedTime");
  return CPQ_OK;
}

void cpq_event_release(cpq_event* ev) {
  if (!ev) return;
  if (ev->ev) (void)hipEventDestroy(ev->ev);
  delete ev;
}

// ---------------------------------------------------------------------------
// Quantization descriptor (quantization.rs:86-153)
// ---------------------------------------------------------------------------

cpq_status cpq_quantization_validate(uint32_t bits, uint32_t group_size) {
  if (!(bits == 2 || bits == 3 || bits == 4 || bits == 5 || bits == 6 || bits == 8))
    return fail(CPQ_ERR_INVALID_ARGUMENT, "unsupported quantization bits " + std::to_string(bits) +
                                              " - expected one of [2, 3, 4, 5, 6, 8]");
  if (group_size == 0 || (group_size & (group_size - 1)) != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "group_size " + std::to_string(group_size) + " must be a positive power of two");
  uint64_t group_bits = uint64_t(group_size) * bits;
  if (group_bits % 32 != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "group_size " + std::to_string(group_size) + " x bits " +
                                              std::to_string(bits) + " = " +
                                              std::to_string(group_bits) +
                                              " bits per group does not fit in whole u32 words");
  return CPQ_OK;
}

cpq_status cpq_packed_word_count(uint32_t bits, uint32_t group_size, size_t scalar_count,
                                 size_t* out) {
  cpq_status st = cpq_quantization_validate(bits, group_size);
  if (st != CPQ_OK) return st;
  if (scalar_count % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "scalar_count " + std::to_string(scalar_count) +
                                              " is not divisible by group_size " +
                                              std::to_string(group_size));
  if (scalar_count > SIZE_MAX / bits)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "scalar_count " + std::to_string(scalar_count) +
                                              " x bits " + std::to_string(bits) + " overflows");
  if (out) *out = scalar_count * bits / 32;
  return CPQ_OK;
}

cpq_status cpq_group_count(uint32_t bits, uint32_t group_size, size_t scalar_count, size_t* out) {
  cpq_status st = cpq_quantization_validate(bits, group_size);
  if (st != CPQ_OK) return st;
  if (scalar_count % group_size != 0)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "scalar_count " + std::to_string(scalar_count) +
                                              " is not divisible by group_size " +
                                              std::to_string(group_size));
  if (out) *out = scalar_count / group_size;
  return CPQ_OK;
}

int cpq_kernel_available(cpq_dtype dtype, uint32_t group_size, uint32_t bits) {
  return cpq::kernel_available(dtype, group_size, bits) ? 1 : 0;
}

}  // extern "C"
