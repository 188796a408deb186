// Device-side building blocks shared by the verify-path kernels (gfx950 / CDNA4).
//
// Packed-weight layout (same bytes the reference consumes, restated from
// dflash_mlx/verify_qmm.py:97-115, 243-249): w_q uint32 [N, K/8], word j of
// row n holds k = 8j .. 8j+7, nibble i at bits 4i; scales / biases
// [N, K/gs] in the activation dtype.
//
// Arithmetic scheme.  For one quantisation group g of row n,
//     sum_k x[m,k] (q[n,k] s + b) = s * sum_k x[m,k] (OFF + q[n,k]) + (b - OFF s) * X[m,g]
// with X[m,g] = sum_{k in g} x[m,k].  The bracket (OFF + q) is produced with
// one AND-OR per pair of nibbles: (w & 0x000F000F) | MAGIC is a packed pair of
// bf16 values 128+q (exponent 2^7, q in the low mantissa bits; f16 uses 1024+q),
// exact, and feeds v_mfma_f32_16x16x32_{bf16,f16} directly.  The per-group
// scale is applied to the fp32 MFMA result, and the bias term is one
// v_mfma_f32_16x16x4_f32 per four groups (X in the A operand, b - OFF s in the
// B operand).  Every product is exact and every sum is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dfmi {

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;

struct BF16 {};
struct F16 {};

template <typename Tag> struct Num;

template <> struct Num<BF16> {
  // bf16 0x4300 == 128.0; OR-ing a nibble into the low mantissa bits gives 128 + q.
  static constexpr uint32_t MAGIC = 0x43004300u;
  static constexpr uint32_t ONE2 = 0x3F803F80u;  // (1.0, 1.0)
  static constexpr float OFF = 128.0f;
  __device__ static inline float lo(uint32_t u) { return __uint_as_float(u << 16); }
  __device__ static inline float hi(uint32_t u) { return __uint_as_float(u & 0xFFFF0000u); }
  __device__ static inline float h2f(uint32_t h) { return __uint_as_float(h << 16); }
  __device__ static inline uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (__bf16)f); }
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

template <> struct Num<F16> {
  // f16 0x6400 == 1024.0; 0x6400 | q == 1024 + q.
  static constexpr uint32_t MAGIC = 0x64006400u;
  static constexpr uint32_t ONE2 = 0x3C003C00u;
  static constexpr float OFF = 1024.0f;
  __device__ static inline float lo(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u & 0xFFFFu));
  }
  __device__ static inline float hi(uint32_t u) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(u >> 16));
  }
  __device__ static inline float h2f(uint32_t h) { return lo(h); }
  __device__ static inline uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }
  __device__ static inline f32x4 mma(u32x4 a, u32x4 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

// One packed word (8 nibbles q0..q7) -> MFMA operand of 8 16-bit values in the
// order (q0,q4, q1,q5, q2,q6, q3,q7), each value OFF + q.
template <typename Tag>
__device__ inline u32x4 dequant_word4(uint32_t w) {
  constexpr uint32_t M = Num<Tag>::MAGIC;
  u32x4 r;
  r.x = (w & 0x000F000Fu) | M;
  r.y = ((w >> 4) & 0x000F000Fu) | M;
  r.z = ((w >> 8) & 0x000F000Fu) | M;
  r.w = ((w >> 12) & 0x000F000Fu) | M;
  return r;
}

// 8 consecutive activations (x0..x7 as four packed pairs) -> the same element
// order as dequant_word4: (x0,x4, x1,x5, x2,x6, x3,x7).
__device__ inline u32x4 permute_x8(u32x4 v) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(v.z, v.x, 0x05040100u);
  r.y = __builtin_amdgcn_perm(v.z, v.x, 0x07060302u);
  r.z = __builtin_amdgcn_perm(v.w, v.y, 0x05040100u);
  r.w = __builtin_amdgcn_perm(v.w, v.y, 0x07060302u);
  return r;
}

__device__ inline f32x4 mma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ inline f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Monotone map float -> uint32 (larger float -> larger key); NaN maps to 0 so
// it never wins an argmax unless every candidate is NaN.
__device__ inline uint32_t ordered_key(float v) {
  uint32_t u = __float_as_uint(v);
  if (v != v) return 0u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// 64-bit argmax key: value first, then the lower index.
__device__ inline unsigned long long argmax_key(float v, uint32_t idx) {
  return ((unsigned long long)ordered_key(v) << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

__device__ inline uint32_t key_index(unsigned long long key) {
  return 0xFFFFFFFFu - (uint32_t)(key & 0xFFFFFFFFull);
}

}  // namespace dfmi
