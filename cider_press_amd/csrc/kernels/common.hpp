// Device-side building blocks shared by the gfx950 kernels.
//
// Packing (reference: kernels-mlx/mlx/backend/metal/kernels/quantized.h:2543-2603):
// element i of a weight row occupies bits [bits*i, bits*(i+1)) of the row's
// little-endian bit stream, so 32 consecutive elements of a row always occupy
// exactly `bits` consecutive uint32 words ("a chunk").  K is a multiple of the
// group size (>= 32), so a chunk never straddles a group or a row.
//
// Dequantization contract: w = RNE_T(fmaf(scale, q, bias)) -- one fp32
// rounding (s*q is exact in fp32) followed by one rounding to T.  Every
// kernel feeds these T-rounded weights to its dot products, so all paths
// agree with the dequantize op bit for bit on the weights themselves.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cpq {
namespace dev {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct BF16 {
  static __device__ __forceinline__ float to_f32(uint16_t h) {
    return __uint_as_float(uint32_t(h) << 16);
  }
  // Two f32 -> packed T pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f32x2 v = {lo, hi};
    bf16x2 r = __builtin_convertvector(v, bf16x2);
    return __builtin_bit_cast(uint32_t, r);
  }
  static __device__ __forceinline__ uint16_t from_f32(float v) {
    return __builtin_bit_cast(uint16_t, (__bf16)v);
  }
  // Low / high element of a packed pair as f32.
  static __device__ __forceinline__ float lo(uint32_t p) { return __uint_as_float(p << 16); }
  static __device__ __forceinline__ float hi(uint32_t p) { return __uint_as_float(p & 0xffff0000u); }
  // fp32 += a.lo*b.lo + a.hi*b.hi (v_dot2_f32_bf16; products of two T are exact in fp32).
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, a),
                                           __builtin_bit_cast(bf16x2, b), c, false);
  }
};

struct F16 {
  static __device__ __forceinline__ float to_f32(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
  }
  static __device__ __forceinline__ uint32_t pack2(float lo, float hi) {
    f32x2 v = {lo, hi};
    f16x2 r = __builtin_convertvector(v, f16x2);
    return __builtin_bit_cast(uint32_t, r);
  }
  static __device__ __forceinline__ uint16_t from_f32(float v) {
    return __builtin_bit_cast(uint16_t, (_Float16)v);
  }
  static __device__ __forceinline__ float lo(uint32_t p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p & 0xffffu));
  }
  static __device__ __forceinline__ float hi(uint32_t p) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(p >> 16));
  }
  static __device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c,
                                  false);
  }
};

// Hide a value's known bits from the optimiser so a byte conversion of a
// masked word stays one v_and + v_cvt_f32_ubyteN instead of being re-derived
// as a bit-field extract per element.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
  asm volatile("" : "+v"(v));
  return v;
}

// Byte j of a word, as f32 (selects v_cvt_f32_ubyte{0..3}).
template <int J>
__device__ __forceinline__ float ubyte_f32(uint32_t w) {
  return (float)((w >> (8 * J)) & 0xffu);
}

// Element E (0..31) of a chunk held in `bits` words, as an unsigned integer.
template <int BITS, int E>
__device__ __forceinline__ uint32_t chunk_elem(const uint32_t* w) {
  constexpr int bit = BITS * E;
  constexpr int wi = bit >> 5;
  constexpr int off = bit & 31;
  constexpr uint32_t mask = (1u << BITS) - 1u;
  if constexpr (off + BITS <= 32) {
    return (w[wi] >> off) & mask;
  } else {
    // straddles two words: funnel shift (v_alignbit_b32)
    return (uint32_t)((((uint64_t)w[wi + 1] << 32) | w[wi]) >> off) & mask;
  }
}

// Dequantize 8 consecutive elements [8*P, 8*P+8) of a chunk into 4 packed T
// pairs (natural order: pair i = elements 2i, 2i+1).  `s16` = scale/16
// (exact), used where the nibble is read in place as 16*q.
template <typename TT, int BITS, int P>
__device__ __forceinline__ void dequant8(const uint32_t* w, float s, float s16, float b,
                                         uint32_t* out) {
  if constexpr (BITS == 4) {
    // One word holds the 8 nibbles.  lo bytes = even nibbles q, hi bytes =
    // odd nibbles as 16*q; s16*(16q) == s*q exactly.
    const uint32_t word = w[P];
    const uint32_t lo = opaque(word & 0x0F0F0F0Fu);
    const uint32_t hi = opaque(word & 0xF0F0F0F0u);
    out[0] = TT::pack2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s16, ubyte_f32<0>(hi), b));
    out[1] = TT::pack2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s16, ubyte_f32<1>(hi), b));
    out[2] = TT::pack2(fmaf(s, ubyte_f32<2>(lo), b), fmaf(s16, ubyte_f32<2>(hi), b));
    out[3] = TT::pack2(fmaf(s, ubyte_f32<3>(lo), b), fmaf(s16, ubyte_f32<3>(hi), b));
  } else if constexpr (BITS == 8) {
    const uint32_t w0 = w[2 * P], w1 = w[2 * P + 1];
    out[0] = TT::pack2(fmaf(s, ubyte_f32<0>(w0), b), fmaf(s, ubyte_f32<1>(w0), b));
    out[1] = TT::pack2(fmaf(s, ubyte_f32<2>(w0), b), fmaf(s, ubyte_f32<3>(w0), b));
    out[2] = TT::pack2(fmaf(s, ubyte_f32<0>(w1), b), fmaf(s, ubyte_f32<1>(w1), b));
    out[3] = TT::pack2(fmaf(s, ubyte_f32<2>(w1), b), fmaf(s, ubyte_f32<3>(w1), b));
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      // generic bit widths: explicit extraction per element
      float q0, q1;
      switch (i) {
        case 0: q0 = (float)chunk_elem<BITS, 8 * P + 0>(w); q1 = (float)chunk_elem<BITS, 8 * P + 1>(w); break;
        case 1: q0 = (float)chunk_elem<BITS, 8 * P + 2>(w); q1 = (float)chunk_elem<BITS, 8 * P + 3>(w); break;
        case 2: q0 = (float)chunk_elem<BITS, 8 * P + 4>(w); q1 = (float)chunk_elem<BITS, 8 * P + 5>(w); break;
        default: q0 = (float)chunk_elem<BITS, 8 * P + 6>(w); q1 = (float)chunk_elem<BITS, 8 * P + 7>(w); break;
      }
      out[i] = TT::pack2(fmaf(s, q0, b), fmaf(s, q1, b));
    }
  }
}

// Whole 32-element chunk -> 16 packed T pairs.
template <typename TT, int BITS>
__device__ __forceinline__ void dequant_chunk(const uint32_t* w, float s, float b, uint32_t* out) {
  const float s16 = s * 0.0625f;
  dequant8<TT, BITS, 0>(w, s, s16, b, out + 0);
  dequant8<TT, BITS, 1>(w, s, s16, b, out + 4);
  dequant8<TT, BITS, 2>(w, s, s16, b, out + 8);
  dequant8<TT, BITS, 3>(w, s, s16, b, out + 12);
}

// Load the `BITS` words of chunk c of a row (global memory, 4-byte aligned).
template <int BITS>
__device__ __forceinline__ void load_chunk(const uint32_t* __restrict__ row, size_t c, uint32_t* w) {
  const uint32_t* p = row + c * BITS;
  if constexpr (BITS == 4) {
    u32x4 v = *reinterpret_cast<const u32x4*>(p);
    w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
  } else if constexpr (BITS == 8) {
    u32x4 v0 = *reinterpret_cast<const u32x4*>(p);
    u32x4 v1 = *reinterpret_cast<const u32x4*>(p + 4);
    w[0] = v0.x; w[1] = v0.y; w[2] = v0.z; w[3] = v0.w;
    w[4] = v1.x; w[5] = v1.y; w[6] = v1.z; w[7] = v1.w;
  } else if constexpr (BITS == 2) {
    u32x2 v = *reinterpret_cast<const u32x2*>(p);
    w[0] = v.x; w[1] = v.y;
  } else {
#pragma unroll
    for (int i = 0; i < BITS; ++i) w[i] = p[i];
  }
}

// Wave64 sum via DPP-friendly butterfly.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace dev
}  // namespace cpq
