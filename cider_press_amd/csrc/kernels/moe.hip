// Routed-expert plumbing around gather_qmm for gfx950: the router's top-k
// selection, the sort of (token, slot) rows by expert that gather_qmm's
// sorted form consumes, and the weighted combine back to tokens.
//
// Reference: the reference names this feature but has not built it
// (docs/inference/feed-forward.md:98-107, 131-137: router scores, top-k
// experts per token, gather_qmm dispatch, loop-or-fuse).  The kernel it would
// feed is MLX's affine_gather_qmm_rhs (quantized.h:2242-2436), which expects
// rows sorted by expert.  The semantics here are the usual ones for that
// pipeline, stated exactly so they can be tested:
//   route:   p = softmax(logits[t, :]) in fp32; the k largest p (ties: lower
//            expert index first), in descending order; with `normalize`
//            they are divided by their sum.
//   sort:    rows r = t*k + j ordered by expert, stably (equal experts keep
//            row order) -- a stable argsort of the flattened expert ids.
//            lhs[p] = token of the row at sorted position p, rhs[p] = its
//            expert, inv[r] = the sorted position of row r, offsets[e] =
//            first sorted position of expert e (offsets[E] = T*k).
//   combine: out[t, :] = RNE_T(sum_j scores[t*k + j] * y[inv[t*k + j], :]),
//            fp32, j ascending.
// All three are tiny next to the expert matmuls (bytes: T*E logits;
// 16*T*k of indices; (k + 1)*T*N*sizeof(T) for the combine).
#include "../cpq_internal.hpp"
#include "common.hpp"

namespace cpq {
namespace {

using namespace dev;

constexpr int kMaxExperts = 1024;
constexpr int kMaxTopK = 16;
constexpr int kSortRows = 256;  // rows per sort block (four waves of 64)

template <int L>
__device__ __forceinline__ float logit_at(const void* p, size_t i) {
  if constexpr (L == 0) return static_cast<const float*>(p)[i];
  else if constexpr (L == 1) return F16::to_f32(static_cast<const uint16_t*>(p)[i]);
  else return BF16::to_f32(static_cast<const uint16_t*>(p)[i]);
}

// Wave-wide reductions of the device library (DPP row shifts, no LDS).
extern "C" __device__ float __ockl_wfred_max_f32(float);
extern "C" __device__ float __ockl_wfred_add_f32(float);
extern "C" __device__ unsigned long long __ockl_wfred_max_u64(unsigned long long);

// Ranking key of (p, e) for p >= 0: the float bits order like the values, and
// ~e puts the lower expert first on equal p.  0 means "nothing left".
__device__ __forceinline__ unsigned long long rank_key(float p, int e) {
  return ((unsigned long long)__float_as_uint(p) << 32) | (uint32_t)~(uint32_t)e;
}

// One wave per token.  Lane l holds experts l + 64 i, i < NV (NV = ceil(E/64)).
template <int L, int NV>
__global__ __launch_bounds__(256) void route_kernel(const void* __restrict__ logits, int tokens, int n_experts,
                                                    int top_k, int normalize, uint32_t* __restrict__ experts,
                                                    float* __restrict__ scores) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= tokens) return;  // whole waves leave together
  const size_t row = (size_t)t * n_experts;
  float v[NV];
  bool live[NV];
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int e = lane + 64 * i;
    live[i] = e < n_experts;
    v[i] = live[i] ? logit_at<L>(logits, row + e) : -INFINITY;
    m = fmaxf(m, v[i]);
  }
  m = __ockl_wfred_max_f32(m);
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    v[i] = live[i] ? expf(v[i] - m) : 0.f;
    sum += v[i];
  }
  const float inv = 1.f / __ockl_wfred_add_f32(sum);
#pragma unroll
  for (int i = 0; i < NV; ++i) v[i] *= inv;

  // Lane j keeps pick j (top_k <= 16 < 64 lanes).
  float my_p = 0.f;
  int my_e = 0;
  for (int j = 0; j < top_k; ++j) {
    unsigned long long best = 0ull;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
      const unsigned long long key = live[i] ? rank_key(v[i], lane + 64 * i) : 0ull;
      best = key > best ? key : best;
    }
    best = __ockl_wfred_max_u64(best);
    const int be = (int)~(uint32_t)best;
    const float bp = __uint_as_float((uint32_t)(best >> 32));
    // The owner retires the winner.
    if ((be & 63) == lane) {
#pragma unroll
      for (int i = 0; i < NV; ++i)
        if (i == (be >> 6)) live[i] = false;
    }
    if (lane == j) {
      my_p = bp;
      my_e = be;
    }
  }
  // The picks' sum in pick order (lane 0 .. k-1), the order a serial loop uses.
  float psum = 0.f;
  for (int j = 0; j < top_k; ++j) psum += __shfl(my_p, j, 64);
  if (lane < top_k) {
    experts[(size_t)t * top_k + lane] = (uint32_t)my_e;
    scores[(size_t)t * top_k + lane] = normalize ? my_p / psum : my_p;
  }
}

// Per-block expert histograms: counts[b * E + e].
__global__ __launch_bounds__(64) void sort_count_kernel(const uint32_t* __restrict__ experts, int rows, int n_experts,
                                                        uint32_t* __restrict__ counts) {
  __shared__ uint32_t h[kMaxExperts];
  for (int e = threadIdx.x; e < n_experts; e += 64) h[e] = 0u;
  __syncthreads();
  const int r0 = blockIdx.x * kSortRows;
  for (int r = r0 + threadIdx.x; r < min(rows, r0 + kSortRows); r += 64) atomicAdd(&h[experts[r]], 1u);
  __syncthreads();
  for (int e = threadIdx.x; e < n_experts; e += 64) counts[(size_t)blockIdx.x * n_experts + e] = h[e];
}

// Thread e turns the histograms into per-(block, expert) start positions
// (expert-major, block order within an expert) and writes offsets[e];
// thread E-1 also writes offsets[E].  One block of 1024 threads.
__global__ __launch_bounds__(1024) void sort_scan_kernel(uint32_t* __restrict__ counts, int blocks, int n_experts,
                                                         uint32_t* __restrict__ offsets) {
  __shared__ uint32_t tot[kMaxExperts];
  const int e = threadIdx.x;
  uint32_t s = 0;
  if (e < n_experts) {
#pragma unroll 8
    for (int b = 0; b < blocks; ++b) s += counts[(size_t)b * n_experts + e];
  }
  tot[e] = e < n_experts ? s : 0u;
  __syncthreads();
  // Exclusive prefix over experts (Hillis-Steele in LDS; E <= 1024).
  for (int d = 1; d < kMaxExperts; d <<= 1) {
    const uint32_t add = e >= d ? tot[e - d] : 0u;
    __syncthreads();
    tot[e] += add;
    __syncthreads();
  }
  if (e < n_experts) {
    uint32_t start = tot[e] - s;  // exclusive
    offsets[e] = start;
#pragma unroll 8
    for (int b = 0; b < blocks; ++b) {
      const uint32_t c = counts[(size_t)b * n_experts + e];
      counts[(size_t)b * n_experts + e] = start;
      start += c;
    }
    if (e == n_experts - 1) offsets[n_experts] = start;
  }
}

// Four waves per block of kSortRows rows, wave w on rows 64w .. 64w+63 of
// the block.  A lane's rank among the earlier lanes of its wave with the same
// expert comes from 64 lane reads (no LDS round trips); the last lane of each
// (wave, expert) run publishes the run's length, and a lane's sorted position
// is its block's start for the expert, plus the counts of the earlier waves,
// plus its rank -- so equal experts keep row order.
__global__ __launch_bounds__(256) void sort_scatter_kernel(const uint32_t* __restrict__ experts, int rows, int top_k,
                                                           int n_experts, const uint32_t* __restrict__ starts,
                                                           uint32_t* __restrict__ lhs, uint32_t* __restrict__ rhs,
                                                           uint32_t* __restrict__ inv) {
  __shared__ uint32_t cnt[4][kMaxExperts];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int i = threadIdx.x; i < 4 * kMaxExperts; i += 256) (&cnt[0][0])[i] = 0u;
  const int r = blockIdx.x * kSortRows + threadIdx.x;
  const bool live = r < rows;
  const uint32_t e = live ? experts[r] : 0xffffffffu;
  uint32_t rank = 0, same = 0;
#pragma unroll 8
  for (int i = 0; i < 64; ++i) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)e, i);
    const uint32_t eq = (o == e) ? 1u : 0u;
    same += eq;
    rank += (i < lane) ? eq : 0u;
  }
  __syncthreads();  // cnt cleared
  if (live && rank + 1 == same) cnt[wave][e] = same;
  __syncthreads();
  if (live) {
    uint32_t pos = starts[(size_t)blockIdx.x * n_experts + e] + rank;
    for (int w = 0; w < wave; ++w) pos += cnt[w][e];
    lhs[pos] = (uint32_t)(r / top_k);
    rhs[pos] = e;
    inv[r] = pos;
  }
}

// out[t, c..c+7] = sum_j scores[t*k+j] * y[inv[t*k+j], c..c+7]; one thread per 8 columns.
// A position at or past rows (a corrupted inv) contributes nothing and is
// counted in *bad once per (token, slot).
template <typename TT>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* __restrict__ y, const float* __restrict__ scores,
                                                      const uint32_t* __restrict__ inv, int tokens, int top_k, int n,
                                                      uint16_t* __restrict__ out, unsigned int* bad) {
  const int per_row = n / 8;
  const size_t total = (size_t)tokens * per_row;
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += stride) {
    const size_t t = i / per_row;
    const int c = (int)(i - t * per_row) * 8;
    float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    const uint32_t rows = (uint32_t)tokens * (uint32_t)top_k;
    for (int j = 0; j < top_k; ++j) {
      const uint32_t p = inv[t * top_k + j];
      if (p >= rows) {
        if (c == 0) atomicAdd(bad, 1u);
        continue;
      }
      const float w = scores[t * top_k + j];
      const u32x4 v = *reinterpret_cast<const u32x4*>(y + (size_t)p * n + c);
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        acc[2 * h] = fmaf(w, TT::to_f32((uint16_t)(v[h] & 0xffffu)), acc[2 * h]);
        acc[2 * h + 1] = fmaf(w, TT::to_f32((uint16_t)(v[h] >> 16)), acc[2 * h + 1]);
      }
    }
    u32x4 o;
#pragma unroll
    for (int h = 0; h < 4; ++h) o[h] = TT::pack2(acc[2 * h], acc[2 * h + 1]);
    *reinterpret_cast<u32x4*>(out + t * n + c) = o;
  }
}

}  // namespace

size_t moe_sort_scratch_bytes(int rows, int n_experts) {
  const size_t blocks = (size_t)(rows + kSortRows - 1) / kSortRows;
  return blocks * (size_t)n_experts * 4;
}

template <int L>
hipError_t launch_route_nv(hipStream_t s, const void* logits, int tokens, int n_experts, int top_k, int normalize,
                           uint32_t* experts, float* scores) {
  const unsigned grid = (unsigned)((tokens + 3) / 4);
  const int nv = (n_experts + 63) / 64;
#define CPQ_ROUTE(NVV) \
  hipLaunchKernelGGL((route_kernel<L, NVV>), dim3(grid), dim3(256), 0, s, logits, tokens, n_experts, top_k, \
                     normalize, experts, scores)
  if (nv <= 1) CPQ_ROUTE(1);
  else if (nv <= 2) CPQ_ROUTE(2);
  else if (nv <= 4) CPQ_ROUTE(4);
  else if (nv <= 8) CPQ_ROUTE(8);
  else CPQ_ROUTE(16);
#undef CPQ_ROUTE
  return hipGetLastError();
}

hipError_t launch_moe_route(hipStream_t s, int logits_dtype, const void* logits, int tokens, int n_experts, int top_k,
                            int normalize, uint32_t* experts, float* scores) {
  if (tokens == 0) return hipSuccess;
  if (logits_dtype == CPQ_DTYPE_F32)
    return launch_route_nv<0>(s, logits, tokens, n_experts, top_k, normalize, experts, scores);
  if (logits_dtype == CPQ_DTYPE_F16)
    return launch_route_nv<1>(s, logits, tokens, n_experts, top_k, normalize, experts, scores);
  return launch_route_nv<2>(s, logits, tokens, n_experts, top_k, normalize, experts, scores);
}

hipError_t launch_moe_sort(hipStream_t s, const uint32_t* experts, int rows, int top_k, int n_experts,
                           uint32_t* scratch, uint32_t* lhs, uint32_t* rhs, uint32_t* inv, uint32_t* offsets) {
  const int blocks = (rows + kSortRows - 1) / kSortRows;
  if (blocks == 0) {
    hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, s, scratch, 0, n_experts, offsets);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(sort_count_kernel, dim3((unsigned)blocks), dim3(64), 0, s, experts, rows, n_experts, scratch);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, s, scratch, blocks, n_experts, offsets);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(sort_scatter_kernel, dim3((unsigned)blocks), dim3(256), 0, s, experts, rows, top_k, n_experts,
                     scratch, lhs, rhs, inv);
  return hipGetLastError();
}

hipError_t launch_moe_combine(hipStream_t s, int dtype, const void* y, const float* scores, const uint32_t* inv,
                              int tokens, int top_k, int n, void* out, unsigned int* bad) {
  const size_t total = (size_t)tokens * (n / 8);
  if (total == 0) return hipSuccess;
  size_t blocks = (total + 255) / 256;
  if (blocks > 256 * 32) blocks = 256 * 32;
  if (dtype == CPQ_DTYPE_BF16)
    hipLaunchKernelGGL(combine_kernel<BF16>, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const uint16_t*>(y), scores, inv, tokens, top_k, n, static_cast<uint16_t*>(out), bad);
  else
    hipLaunchKernelGGL(combine_kernel<F16>, dim3((unsigned)blocks), dim3(256), 0, s,
                       static_cast<const uint16_t*>(y), scores, inv, tokens, top_k, n, static_cast<uint16_t*>(out), bad);
  return hipGetLastError();
}

}  // namespace cpq
