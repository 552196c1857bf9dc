// cpq_affine_qmm_t_noalloc: the prefill op for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, hosts
// that forbid allocation after start-up).  Same validation, kernel choice and
// numerics as cpq_affine_qmm_t on a session with the default scratch
// capacity, but on a caller's hipStream_t and with no session: the split-K
// arrival counters and fp32 partial tiles live in `scratch`, a file-scope
// device array of kNoAllocScratchBytes that every GPU the library runs on
// holds until the process ends.
//
// Nothing here allocates: the array's per-device address comes from
// hipGetSymbolAddress (once per device, with that device current), the CU
// count from hipDeviceGetAttribute, and the kernels are launched exactly as
// for a session.  A shape whose kernel choice needs more scratch than the
// array holds is refused with CPQ_ERR_BUFFER_TOO_LARGE before any launch.
//
// Sharing: every call on a GPU uses that GPU's one array.  The arrival
// counters start at zero (module load, and explicitly at set-up) and every
// launch that completes leaves the counters it used at zero again; the
// partial tiles are written before they are read within a launch.  Calls
// that overlap on one GPU (two streams, or two host threads) race on the
// array and must be serialised by the caller.
#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

#include "cpq_internal.hpp"

namespace cpq {
namespace {

// 16 MiB of partial tiles (256 fp32 tiles of 128 x 128: the config 3a split)
// behind the 64 KiB of arrival counters.
constexpr size_t kNoAllocScratchBytes = kWideCounterBytes + (size_t(16) << 20);
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct DeviceSlot {
  std::once_flag once;
  hipError_t status = hipSuccess;
  void* ptr = nullptr;  // device address of `scratch` on this device
  int cu_count = 0;
};
DeviceSlot g_slots[kMaxDevices];

// Per-device set-up on the first call with that device current: the array's
// address on this device, its counters cleared (a kernel, so a stream that is
// being captured records no memset), the CU count.
hipError_t device_slot(hipStream_t stream, DeviceSlot** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  DeviceSlot& slot = g_slots[dev];
  std::call_once(slot.once, [&] {
    void* p = nullptr;
    hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r == hipSuccess) r = hipDeviceGetAttribute(&slot.cu_count, hipDeviceAttributeMultiprocessorCount, dev);
    // The array is zero from module load; the clear re-establishes that
    // explicitly.  Under graph capture it is recorded as a kernel node that
    // runs ahead of the op at every replay, which is equally correct.
    if (r == hipSuccess) r = zero_words(stream, p, kWideCounterBytes / 4);
    if (r == hipSuccess) slot.ptr = p;
    slot.status = r;
  });
  if (slot.status != hipSuccess) return slot.status;
  *out = &slot;
  return hipSuccess;
}

}  // namespace
}  // namespace cpq

using cpq::fail;

extern "C" cpq_status cpq_affine_qmm_t_noalloc(void* hip_stream, cpq_dtype dtype, const uint32_t* w_q,
                                                size_t w_q_len, const void* scales, size_t scales_len,
                                                const void* biases, size_t biases_len, const void* x, size_t x_len,
                                                void* y, size_t y_len, size_t m, size_t n, size_t k,
                                                uint32_t group_size, uint32_t bits) {
  cpq_status st = cpq_check_qmm_args(dtype, w_q_len, scales_len, biases_len, x_len, y_len, m, n, k, group_size, bits);
  if (st != CPQ_OK) return st;
  if (!w_q || !scales || !biases || !x || !y)
    return fail(CPQ_ERR_INVALID_ARGUMENT, "affine_qmm_t_noalloc: NULL buffer");
  if (((reinterpret_cast<uintptr_t>(w_q) | reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(y)) & 15u) ||
      ((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(biases)) & 1u))
    return fail(CPQ_ERR_INVALID_ARGUMENT,
                "affine_qmm_t_noalloc: w_q, x and y must be 16-byte aligned; scales/biases 2-byte");
  hipStream_t stream = static_cast<hipStream_t>(hip_stream);
  cpq::DeviceSlot* slot = nullptr;
  hipError_t e = cpq::device_slot(stream, &slot);
  if (e != hipSuccess) return cpq::hip_fail(e, "affine_qmm_t_noalloc: static scratch set-up");
  const cpq::QuantArgs q{w_q, scales, biases, (int)group_size, (int)bits, dtype};
  // The kernel a session with the default scratch capacity would run; the
  // static array must hold what that kernel uses.
  const cpq::QmmPlan plan =
      cpq::qmm_plan(q, (int)m, (int)n, (int)k, slot->cu_count, cpq::kDefaultSessionScratchBytes);
  if (plan.scratch_bytes > cpq::kNoAllocScratchBytes)
    return fail(CPQ_ERR_BUFFER_TOO_LARGE,
                "affine_qmm_t_noalloc: M=" + std::to_string(m) + ", N=" + std::to_string(n) + ", K=" +
                    std::to_string(k) + " runs a K split of " + std::to_string(plan.split) + " whose partial tiles need " +
                    std::to_string(plan.scratch_bytes) + " bytes of scratch; the static scratch holds " +
                    std::to_string(cpq::kNoAllocScratchBytes) + " (use cpq_affine_qmm_t on a session)");
  e = cpq::launch_qmm(stream, plan, slot->ptr, q, x, y, (int)m, (int)n, (int)k);
  if (e != hipSuccess) return cpq::hip_fail(e, "affine_qmm_t_noalloc launch");
  return CPQ_OK;
}
