// Plain streaming read of up to four device regions in one launch: the HBM
// ceiling that a single kernel of a given byte count reaches on this device,
// timed by the benchmark beside the kernels it bounds over the same rotated
// buffers.  Measurement support only (the reference times its kernels against
// the device's spec bandwidth, crates/cider-press-kernels/tests/
// qmv_dispatch_bench.rs:37-79; this gives the achievable figure instead).
//
// Each workgroup reads a contiguous span of the regions' concatenation with
// 16-byte loads; the XOR of everything read is compared with a value it
// cannot equal in practice, so the loads stay live while nothing is written.
// Several designs are compiled so the ceiling is the best of them, not one
// untuned loop: workgroup size (256 / 512 / 1024 threads), loads in flight
// per lane (4 / 8 / 16), plain or non-temporal loads, and global or buffer
// addressing.
#include "../cpq_internal.hpp"

namespace cpq {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct ReadRegions {
  const u32x4* p[4];
  uint64_t chunks[4];  // 16-byte chunks per region
  uint64_t start[4];   // first chunk of each region in the concatenation
};

template <bool NT>
__device__ __forceinline__ u32x4 ld(const u32x4* p) {
  if constexpr (NT)
    return __builtin_nontemporal_load(p);
  else
    return *p;
}

template <int THREADS, int UNROLL, bool NT, bool BUF>
__global__ __launch_bounds__(THREADS) void stream_read_kernel(ReadRegions r, uint64_t total, uint64_t per_wg,
                                                              uint32_t* __restrict__ sink) {
  const uint64_t c0 = (uint64_t)blockIdx.x * per_wg;
  const uint64_t c1 = c0 + per_wg < total ? c0 + per_wg : total;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (int g = 0; g < 4; ++g) {
    // The part of region g inside [c0, c1).
    const uint64_t a = r.start[g] > c0 ? r.start[g] : c0;
    const uint64_t e = r.start[g] + r.chunks[g] < c1 ? r.start[g] + r.chunks[g] : c1;
    if (a >= e) continue;
    const u32x4* base = r.p[g] + (a - r.start[g]);
    const uint64_t n = e - a;
    if constexpr (BUF) {
      // Buffer addressing over this workgroup's span (at most 4 GiB - 16 B,
      // which per_wg keeps far below): one descriptor, lane offsets in a
      // VGPR, the step in the scalar offset.
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          const_cast<u32x4*>(base), 0, (int)(uint32_t)(n * 16u), 0x00020000);
      uint32_t i = threadIdx.x;
      for (; (uint64_t)i + (UNROLL - 1) * THREADS < n; i += UNROLL * THREADS) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
          v[u] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, i * 16u, u * THREADS * 16, NT ? 2 : 0));
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
      }
      for (; (uint64_t)i < n; i += THREADS) acc ^= base[i];
    } else {
      uint64_t i = threadIdx.x;
      for (; i + (UNROLL - 1) * THREADS < n; i += UNROLL * THREADS) {
        u32x4 v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = ld<NT>(base + i + u * THREADS);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc ^= v[u];
      }
      for (; i < n; i += THREADS) acc ^= base[i];
    }
  }
  if (acc.x == 0x9E3779B9u && acc.y == 0x7F4A7C15u && acc.z == 0x94D049BBu && acc.w == 0x2545F491u)
    sink[0] = acc.x ^ acc.w;
}

template <int THREADS, int UNROLL, bool NT, bool BUF>
hipError_t launch_variant(hipStream_t s, const ReadRegions& r, uint64_t total, uint32_t* sink, int n_wg) {
  const uint64_t per = (total + (uint64_t)n_wg - 1) / (uint64_t)n_wg;
  hipLaunchKernelGGL((stream_read_kernel<THREADS, UNROLL, NT, BUF>), dim3((unsigned)n_wg), dim3(THREADS), 0, s, r,
                     total, per, sink);
  return hipGetLastError();
}

}  // namespace

int stream_read_variant_count() { return 10; }

hipError_t launch_stream_read(hipStream_t s, const void* const* regions, const size_t* bytes, int n_regions,
                              uint32_t* sink, int n_wg, int variant) {
  ReadRegions r{};
  uint64_t total = 0;
  for (int g = 0; g < 4; ++g) {
    r.p[g] = g < n_regions ? static_cast<const u32x4*>(regions[g]) : nullptr;
    r.chunks[g] = g < n_regions ? bytes[g] / 16 : 0;
    r.start[g] = total;
    total += r.chunks[g];
  }
  if (total == 0) return hipSuccess;
  switch (variant) {
    case 0: return launch_variant<256, 4, false, false>(s, r, total, sink, n_wg);
    case 1: return launch_variant<256, 8, false, false>(s, r, total, sink, n_wg);
    case 2: return launch_variant<256, 16, false, false>(s, r, total, sink, n_wg);
    case 3: return launch_variant<512, 4, false, false>(s, r, total, sink, n_wg);
    case 4: return launch_variant<512, 8, false, false>(s, r, total, sink, n_wg);
    case 5: return launch_variant<1024, 4, false, false>(s, r, total, sink, n_wg);
    case 6: return launch_variant<256, 4, true, false>(s, r, total, sink, n_wg);
    case 7: return launch_variant<256, 8, true, false>(s, r, total, sink, n_wg);
    case 8: return launch_variant<256, 8, false, true>(s, r, total, sink, n_wg);
    case 9: return launch_variant<512, 8, false, true>(s, r, total, sink, n_wg);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace cpq
