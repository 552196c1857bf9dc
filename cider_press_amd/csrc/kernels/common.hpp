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

#include "fastpath.hpp"

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

// ---------------------------------------------------------------------------
// Interleaved-slice dequantization (MFMA B operands).
//
// A "slice" is 8 consecutive elements of a chunk (one word at 4-bit, two at
// 8-bit), i.e. one MFMA operand of 8 elements per lane.  The matrix cores
// only need A and B to agree on which k each operand slot holds, so the
// weights are produced in the order that is cheapest to build and the
// activations are permuted once (when staged) to the same order:
//   4-bit and generic widths: slot pairs (e0,e4) (e1,e5) (e2,e6) (e3,e7)
//   8-bit:                    slot pairs (e0,e2) (e1,e3) (e4,e6) (e5,e7)
//
// Fast path (4/8-bit): a nibble or byte is dropped into the mantissa of an
// f16 "magic" 1024 (bit pattern 0x6400 | q), giving 1024+q exactly (or
// 1024+16q for a nibble left in place in the high half of a byte); one
// v_fma_mix_f32 then computes s*(1024+q) + (b - 1024*s) == fmaf(s, q, b)
// with a single rounding -- exact whenever c0 = b - 1024*s (and, at 4-bit,
// c1 = b - 64*s) is itself exact in fp32.  fast_ok() checks that per group;
// groups that fail take the slow path (explicit byte conversions), which
// produces the same bits.
// ---------------------------------------------------------------------------

__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(m), "v"(c));
  return r;
}

__device__ __forceinline__ float f16lo(uint32_t p) {
  return (float)__builtin_bit_cast(f16x2, p).x;
}
__device__ __forceinline__ float f16hi(uint32_t p) {
  return (float)__builtin_bit_cast(f16x2, p).y;
}

template <typename TT>
struct Sig16;
template <>
struct Sig16<BF16> {
  static constexpr bool bf16 = true;
};
template <>
struct Sig16<F16> {
  static constexpr bool bf16 = false;
};

// True when the single-FMA fast path reproduces fmaf(s, q, b) for every q
// of a group with raw scale / bias patterns sv, bv (fastpath.hpp).
template <typename TT>
__device__ __forceinline__ bool fast_ok_bits(uint32_t sv, uint32_t bv);
template <>
__device__ __forceinline__ bool fast_ok_bits<BF16>(uint32_t sv, uint32_t bv) {
  return fast_ok_bf16(sv, bv);
}
template <>
__device__ __forceinline__ bool fast_ok_bits<F16>(uint32_t sv, uint32_t bv) {
  return fast_ok_f16(sv, bv);
}

// Packed check of two groups per word (sufficient, not necessary: a false
// result sends the caller to fast_ok_bits for the groups it saw).
template <typename TT>
__device__ __forceinline__ void fast_quick_add(FastQuick& a, uint32_t s2, uint32_t b2) {
  if constexpr (Sig16<TT>::bf16) fast_quick_add_bf16(a, s2, b2);
  else fast_quick_add_f16(a, s2, b2);
}
template <typename TT>
__device__ __forceinline__ bool fast_quick_ok(const FastQuick& a) {
  if constexpr (Sig16<TT>::bf16) return fast_quick_ok_bf16(a);
  else return fast_quick_ok_f16(a);
}

// Row key of the 16-slot XOR swizzle of activation rows in LDS: r (0..15)
// with its two 2-bit halves swapped.  A 16-byte MFMA operand read serves
// lanes p, p + 4, ..., p + 60 together (rows p, p + 4, p + 8, p + 12 of a
// 16-row block, 4 lane groups); with key(r) = r those 16 lanes meet in 4
// slots (4 bank-conflict cycles per read), with the swapped key in 16.
__device__ __forceinline__ int swz_key(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// Natural 16-byte activation slice -> interleaved slot order of BITS.
template <int BITS>
__device__ __forceinline__ u32x4 interleave_x(u32x4 v) {
  if constexpr (BITS == 8) {
    return u32x4{__builtin_amdgcn_perm(v.y, v.x, 0x05040100u), __builtin_amdgcn_perm(v.y, v.x, 0x07060302u),
                 __builtin_amdgcn_perm(v.w, v.z, 0x05040100u), __builtin_amdgcn_perm(v.w, v.z, 0x07060302u)};
  } else {
    return u32x4{__builtin_amdgcn_perm(v.z, v.x, 0x05040100u), __builtin_amdgcn_perm(v.z, v.x, 0x07060302u),
                 __builtin_amdgcn_perm(v.w, v.y, 0x05040100u), __builtin_amdgcn_perm(v.w, v.y, 0x07060302u)};
  }
}

// Slice I (0..3) of a 32-element chunk held in `w` (BITS words), dequantized
// to 4 packed T pairs in the interleaved slot order.
template <typename TT, int BITS, bool FAST, int I>
__device__ __forceinline__ u32x4 dequant_slice(const uint32_t* w, float s, float s16, float b, float c0,
                                               float c1) {
  if constexpr (BITS == 4 && FAST) {
    const uint32_t M = 0x64006400u;
    const uint32_t word = w[I];
    const uint32_t w8 = word >> 8;
    const uint32_t p0 = and_or(word, 0x000F000Fu, M);  // (1024+q0, 1024+q4)
    const uint32_t p1 = and_or(word, 0x00F000F0u, M);  // (1024+16q1, 1024+16q5)
    const uint32_t p2 = and_or(w8, 0x000F000Fu, M);    // (1024+q2, 1024+q6)
    const uint32_t p3 = and_or(w8, 0x00F000F0u, M);    // (1024+16q3, 1024+16q7)
    return u32x4{TT::pack2(fmaf(s, f16lo(p0), c0), fmaf(s, f16hi(p0), c0)),
                 TT::pack2(fmaf(s16, f16lo(p1), c1), fmaf(s16, f16hi(p1), c1)),
                 TT::pack2(fmaf(s, f16lo(p2), c0), fmaf(s, f16hi(p2), c0)),
                 TT::pack2(fmaf(s16, f16lo(p3), c1), fmaf(s16, f16hi(p3), c1))};
  } else if constexpr (BITS == 8 && FAST) {
    const uint32_t M = 0x64646464u;
    const uint32_t w0 = w[2 * I], w1 = w[2 * I + 1];
    const uint32_t p0 = __builtin_amdgcn_perm(M, w0, 0x04020400u);  // (1024+e0, 1024+e2)
    const uint32_t p1 = __builtin_amdgcn_perm(M, w0, 0x04030401u);  // (1024+e1, 1024+e3)
    const uint32_t p2 = __builtin_amdgcn_perm(M, w1, 0x04020400u);  // (1024+e4, 1024+e6)
    const uint32_t p3 = __builtin_amdgcn_perm(M, w1, 0x04030401u);  // (1024+e5, 1024+e7)
    return u32x4{TT::pack2(fmaf(s, f16lo(p0), c0), fmaf(s, f16hi(p0), c0)),
                 TT::pack2(fmaf(s, f16lo(p1), c0), fmaf(s, f16hi(p1), c0)),
                 TT::pack2(fmaf(s, f16lo(p2), c0), fmaf(s, f16hi(p2), c0)),
                 TT::pack2(fmaf(s, f16lo(p3), c0), fmaf(s, f16hi(p3), c0))};
  } else if constexpr (BITS == 4) {
    const uint32_t word = w[I];
    const uint32_t lo = opaque(word & 0x0F0F0F0Fu);  // q0 q2 q4 q6
    const uint32_t hi = opaque(word & 0xF0F0F0F0u);  // 16q1 16q3 16q5 16q7
    return u32x4{TT::pack2(fmaf(s, ubyte_f32<0>(lo), b), fmaf(s, ubyte_f32<2>(lo), b)),
                 TT::pack2(fmaf(s16, ubyte_f32<0>(hi), b), fmaf(s16, ubyte_f32<2>(hi), b)),
                 TT::pack2(fmaf(s, ubyte_f32<1>(lo), b), fmaf(s, ubyte_f32<3>(lo), b)),
                 TT::pack2(fmaf(s16, ubyte_f32<1>(hi), b), fmaf(s16, ubyte_f32<3>(hi), b))};
  } else if constexpr (BITS == 8) {
    const uint32_t w0 = w[2 * I], w1 = w[2 * I + 1];
    return u32x4{TT::pack2(fmaf(s, ubyte_f32<0>(w0), b), fmaf(s, ubyte_f32<2>(w0), b)),
                 TT::pack2(fmaf(s, ubyte_f32<1>(w0), b), fmaf(s, ubyte_f32<3>(w0), b)),
                 TT::pack2(fmaf(s, ubyte_f32<0>(w1), b), fmaf(s, ubyte_f32<2>(w1), b)),
                 TT::pack2(fmaf(s, ubyte_f32<1>(w1), b), fmaf(s, ubyte_f32<3>(w1), b))};
  } else {
    // generic widths: explicit extraction, (e_j, e_{j+4}) pairs
    return u32x4{TT::pack2(fmaf(s, (float)chunk_elem<BITS, 8 * I + 0>(w), b), fmaf(s, (float)chunk_elem<BITS, 8 * I + 4>(w), b)),
                 TT::pack2(fmaf(s, (float)chunk_elem<BITS, 8 * I + 1>(w), b), fmaf(s, (float)chunk_elem<BITS, 8 * I + 5>(w), b)),
                 TT::pack2(fmaf(s, (float)chunk_elem<BITS, 8 * I + 2>(w), b), fmaf(s, (float)chunk_elem<BITS, 8 * I + 6>(w), b)),
                 TT::pack2(fmaf(s, (float)chunk_elem<BITS, 8 * I + 3>(w), b), fmaf(s, (float)chunk_elem<BITS, 8 * I + 7>(w), b))};
  }
}

// Natural-order fast dequantization of slice I (elements 8I..8I+7 in order,
// pairs (e0,e1) (e2,e3) ...), for MFMA operands whose A side cannot be
// permuted (activations streamed straight into LDS).  Per byte p: one
// v_perm builds (b_p | 0x6400) in both halves, one AND keeps q_lo in the low
// half and 16*q_hi in the high half: (1024 + q_{2p}, 1024 + 16 q_{2p+1}).
template <typename TT, int BITS, bool FAST, int I>
__device__ __forceinline__ u32x4 dequant_slice_nat(const uint32_t* w, float s, float s16, float b,
                                                   float c0, float c1) {
  if constexpr (BITS == 4 && FAST) {
    const uint32_t M = 0x64646464u;
    const uint32_t word = w[I];
    u32x4 out;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t sel = 0x04000400u | (uint32_t)(p << 16) | (uint32_t)p;  // [b_p, 64, b_p, 64]
      const uint32_t t = __builtin_amdgcn_perm(M, word, sel) & 0x64F0640Fu;
      out[p] = TT::pack2(fmaf(s, f16lo(t), c0), fmaf(s16, f16hi(t), c1));
    }
    return out;
  } else if constexpr (BITS == 8 && FAST) {
    const uint32_t M = 0x64646464u;
    const uint32_t w0 = w[2 * I], w1 = w[2 * I + 1];
    const uint32_t p0 = __builtin_amdgcn_perm(M, w0, 0x04010400u);  // (1024+e0, 1024+e1)
    const uint32_t p1 = __builtin_amdgcn_perm(M, w0, 0x04030402u);  // (1024+e2, 1024+e3)
    const uint32_t p2 = __builtin_amdgcn_perm(M, w1, 0x04010400u);
    const uint32_t p3 = __builtin_amdgcn_perm(M, w1, 0x04030402u);
    return u32x4{TT::pack2(fmaf(s, f16lo(p0), c0), fmaf(s, f16hi(p0), c0)),
                 TT::pack2(fmaf(s, f16lo(p1), c0), fmaf(s, f16hi(p1), c0)),
                 TT::pack2(fmaf(s, f16lo(p2), c0), fmaf(s, f16hi(p2), c0)),
                 TT::pack2(fmaf(s, f16lo(p3), c0), fmaf(s, f16hi(p3), c0))};
  } else {
    uint32_t o[4];
    dequant8<TT, BITS, I>(w, s, s16, b, o);
    return u32x4{o[0], o[1], o[2], o[3]};
  }
}

template <typename TT>
struct Mfma16;
template <>
struct Mfma16<BF16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};
template <>
struct Mfma16<F16> {
  static __device__ __forceinline__ f32x4 run(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// Wait until at most N vector-memory loads of this wave are outstanding
// (loads complete in issue order, so this proves every older load done).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  // s_waitcnt simm16 (gfx9): vmcnt[3:0], expcnt[6:4], lgkmcnt[11:8], vmcnt[5:4] at [15:14].
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Workgroup barrier that orders LDS accesses only.  __syncthreads() also
// waits for every global load and store the wave has in flight (on gfx9
// the vector-memory counter covers both); this one waits for the wave's
// LDS operations, so prefetched operands and stores stay in flight across
// it.  Use it where the barrier protects LDS data alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Wave64 sum via DPP-friendly butterfly.
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

}  // namespace dev
}  // namespace cpq
