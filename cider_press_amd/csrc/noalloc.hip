// cpq_affine_qmm_t_noalloc: the prefill op for callers that cannot allocate
// device memory (code under HIP graph capture, tight serving loops, hosts
// that forbid allocation after start-up).  Same validation and numerics as
// cpq_affine_qmm_t, but on a caller's hipStream_t and with no session: the
// split-K arrival counters and fp32 partial tiles live in `scratch`, a
// file-scope device array of kNoAllocScratchBytes that every GPU the library
// runs on holds until the process ends.
//
// Kernel choice: the kernel (chosen by M, as cpq_affine_qmm_t chooses it)
// and K split a session with the default scratch capacity would run,
// whenever its scratch fits the array (then the output is bit-identical to
// cpq_affine_qmm_t's); otherwise the plan the same planner makes for the
// array's capacity (a smaller K split, or none), which differs from the
// session op only in summation order.
//
// Nothing here allocates: the array's per-device address comes from
// hipGetSymbolAddress (once per device, with that device current), the CU
// count from hipDeviceGetAttribute, and the kernels are launched exactly as
// for a session.  The device is the one the caller's stream belongs to (the
// current device for the null stream).  A set-up failure is not remembered:
// the next call tries again.
//
// Sharing: every call on a GPU uses that GPU's one array.  The arrival
// counters are zero from module load and every launch that completes leaves
// the counters it used at zero again; the partial tiles are written before
// they are read within a launch.  Calls that overlap on one GPU (two streams,
// or two host threads) race on the array and must be serialised by the
// caller.
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
  std::mutex mu;
  bool ready = false;
  void* ptr = nullptr;  // device address of `scratch` on this device
  int cu_count = 0;
};
DeviceSlot g_slots[kMaxDevices];

// The slot of the device `stream` belongs to, set up on first use: the
// array's address on that device (queried with that device current) and its
// CU count.  Nothing is launched: the array is zero from module load.
hipError_t device_slot(hipStream_t stream, DeviceSlot** out) {
  int dev = 0;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  DeviceSlot& slot = g_slots[dev];
  std::lock_guard<std::mutex> lock(slot.mu);
  if (!slot.ready) {
    int cur = 0;
    e = hipGetDevice(&cur);
    if (e != hipSuccess) return e;
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess) return e;
    void* p = nullptr;
    int cus = 0;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e == hipSuccess) e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    if (cur != dev) {
      const hipError_t r = hipSetDevice(cur);
      if (e == hipSuccess) e = r;
    }
    if (e != hipSuccess) return e;  // not remembered: the next call tries again
    slot.ptr = p;
    slot.cu_count = cus;
    slot.ready = true;
  }
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
  // The kernel a session with the default scratch capacity would run (chosen
  // by M as affine_qmm_t chooses it) when its scratch fits the static array;
  // else the plan made for the array's capacity.
  const cpq::ExecCtx ex{stream, slot->cu_count, slot->ptr, cpq::kDefaultSessionScratchBytes,
                        cpq::kNoAllocScratchBytes};
  e = cpq::launch_matmul(ex, q, x, y, (int)m, (int)n, (int)k);
  if (e != hipSuccess) return cpq::hip_fail(e, "affine_qmm_t_noalloc launch");
  return CPQ_OK;
}
