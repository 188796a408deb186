// Device-side building blocks shared by the verify-path kernels (gfx950 / CDNA4).
//
// Packed-weight layout (same bytes the reference consumes, restated from
// dflash_mlx/verify_qmm.py:97-115, 243-249): w_q uint32 [N, K/8], word j of
// row n holds k = 8j .. 8j+7, nibble i at bits 4i; scales / biases
// [N, K/gs] in the activation dtype.
//
// Arithmetic scheme.  For one quantisation group g of row n,
//     sum_k x[m,k] (q[n,k] s + b) = s * sum_k x[m,k] (OFF + q[n,k]) + (b - OFF s) * X[m,g]
// with X[m,g] = sum_{k in g} x[m,k].  The bracket (OFF + q) is produced by bit
// operations: (w & 0x000F000F) | MAGIC is a packed pair of bf16 values 128+q
// (exponent 2^7, q in the low mantissa bits; f16 uses 1024+q), exact, and
// feeds v_mfma_f32_16x16x32_{bf16,f16} directly.  The per-group
// scale is applied to the fp32 MFMA result, and the bias term is one
// v_mfma_f32_16x16x4_f32 per four groups (X in the A operand, b - OFF s in the
// B operand).  Every product is exact and every sum is fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

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

// Dequantisation constants held in registers.  gfx9 VOP3 encodings take no
// literal operand, so with literal constants the compiler splits
// (w & mask) | magic into two VOP2 instructions; with the mask in an SGPR and
// MAGIC in a VGPR (the empty asm statements hide their values) it selects one
// v_and_or_b32.  Plain C rather than an asm v_and_or_b32 keeps the compiler's
// hazard tracking (a VALU write to a VGPR an in-flight MFMA still reads).
struct DqConst {
  uint32_t mask;   // 0x000F000F
  uint32_t magic;  // Num<Tag>::MAGIC
};

template <typename Tag>
__device__ inline DqConst dq_const() {
  DqConst c;
  c.mask = 0x000F000Fu;
  c.magic = Num<Tag>::MAGIC;
  asm volatile("" : "+s"(c.mask));
  asm volatile("" : "+v"(c.magic));
  return c;
}

// One packed word (8 nibbles q0..q7, k order) -> MFMA operand of 8 16-bit
// values OFF + q0 .. OFF + q7 in k order, so the activations feed the MFMA
// unpermuted.  Nine VALU operations (dq = dq_const<Tag>()):
//   lo = (w & 0x000F000F) | MAGIC          -> 16-bit pairs (q0, q4)
//   mi = ((w >> 8) & 0x000F000F) | MAGIC   -> (q2, q6)
//   od = (w >> 4) & 0x0F0F0F0F             -> bytes q1, q3, q5, q7
// and four byte permutes that put an odd nibble byte next to an even one,
// each 16-bit value keeping the MAGIC high byte.
template <typename Tag>
__device__ inline u32x4 dequant_word4(uint32_t w, const DqConst& dq) {
  const uint32_t lo = (w & dq.mask) | dq.magic;
  const uint32_t mi = ((w >> 8) & dq.mask) | dq.magic;
  const uint32_t od = (w >> 4) & 0x0F0F0F0Fu;
  u32x4 r;
  // __builtin_amdgcn_perm(S0, S1, sel): selector byte 0..3 picks a byte of
  // S1, 4..7 a byte of S0.
  r.x = __builtin_amdgcn_perm(od, lo, 0x03040100u);  // (q0, q1)
  r.y = __builtin_amdgcn_perm(od, mi, 0x03050100u);  // (q2, q3)
  r.z = __builtin_amdgcn_perm(od, lo, 0x03060302u);  // (q4, q5)
  r.w = __builtin_amdgcn_perm(od, mi, 0x03070302u);  // (q6, q7)
  return r;
}

// The same word as an MFMA operand in the slot order (q0, q4, q1, q5, q2, q6,
// q3, q7): nibbles 4 apart share a 16-bit pair after one shift, so seven VALU
// operations (three shifts, four v_and_or_b32) and no permutes.  The other
// operand must hold its 8 k in the same order (kperm_x); the MFMA's sum over
// the 32 k of a lane group does not depend on which slot holds which k.
template <typename Tag>
__device__ inline u32x4 dequant_word4_kperm(uint32_t w, const DqConst& dq) {
  u32x4 r;
  r.x = (w & dq.mask) | dq.magic;          // (q0, q4)
  r.y = ((w >> 4) & dq.mask) | dq.magic;   // (q1, q5)
  r.z = ((w >> 8) & dq.mask) | dq.magic;   // (q2, q6)
  r.w = ((w >> 12) & dq.mask) | dq.magic;  // (q3, q7)
  return r;
}

// 8 activations in k order (x0 x1 | x2 x3 | x4 x5 | x6 x7) -> the slot order of
// dequant_word4_kperm (x0 x4 | x1 x5 | x2 x6 | x3 x7): four byte permutes.
__device__ inline u32x4 kperm_x(u32x4 a) {
  u32x4 r;
  r.x = __builtin_amdgcn_perm(a.z, a.x, 0x05040100u);  // (x0, x4)
  r.y = __builtin_amdgcn_perm(a.z, a.x, 0x07060302u);  // (x1, x5)
  r.z = __builtin_amdgcn_perm(a.w, a.y, 0x05040100u);  // (x2, x6)
  r.w = __builtin_amdgcn_perm(a.w, a.y, 0x07060302u);  // (x3, x7)
  return r;
}

// Two words of 8-bit values (q0..q3, q4..q7, k order, lowest byte first)
// -> MFMA operand of 8 16-bit values in k order, exactly:
//   bf16: q -> fp32 (v_cvt_f32_ubyte), whose high half is the bf16 value
//         (q < 256 has at most 8 significant bits); no offset;
//   f16:  one byte permute per pair against the magic 0x6400 high bytes:
//         1024 + q (f16 has 10 mantissa bits); offset 1024.
template <typename Tag>
__device__ inline u32x4 dequant_word8(uint32_t w0, uint32_t w1, const DqConst& dq) {
  u32x4 r;
  if constexpr (std::is_same<Tag, BF16>::value) {
    const uint32_t w[2] = {w0, w1};
    uint32_t d[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float f0 = (float)(w[h] & 0xFFu);
      const float f1 = (float)((w[h] >> 8) & 0xFFu);
      const float f2 = (float)((w[h] >> 16) & 0xFFu);
      const float f3 = (float)(w[h] >> 24);
      // high halves: (f1, f0) and (f3, f2)
      d[2 * h] = __builtin_amdgcn_perm(__float_as_uint(f1), __float_as_uint(f0), 0x07060302u);
      d[2 * h + 1] = __builtin_amdgcn_perm(__float_as_uint(f3), __float_as_uint(f2), 0x07060302u);
    }
    r = u32x4{d[0], d[1], d[2], d[3]};
  } else {
    // selector bytes 0..3 pick bytes of the word, 5 and 7 the magic's 0x64
    r.x = __builtin_amdgcn_perm(dq.magic, w0, 0x07010500u);  // (q0, q1)
    r.y = __builtin_amdgcn_perm(dq.magic, w0, 0x07030502u);  // (q2, q3)
    r.z = __builtin_amdgcn_perm(dq.magic, w1, 0x07010500u);  // (q4, q5)
    r.w = __builtin_amdgcn_perm(dq.magic, w1, 0x07030502u);  // (q6, q7)
  }
  return r;
}

__device__ inline f32x4 mma_f32_16x16x4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ inline f32x4 zero4() { return f32x4{0.f, 0.f, 0.f, 0.f}; }

// Raw buffer resource over [base, base + bytes): word 3 = 0x00020000 (32-bit
// data format, the gfx9 raw-buffer setting); reads at or past `bytes` return
// zero instead of touching memory.
__device__ inline __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

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
