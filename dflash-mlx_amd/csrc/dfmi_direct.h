// Register-direct main loop of the verify-path matmuls (M <= 16).
//
// Every wavefront streams its own weight rows straight into registers: per
// step of 256 k and 16-row tile, a lane loads two 16-byte pieces of its row
// (row = lane & 15, piece kg = lane >> 4 of each 64-byte half), so one load
// instruction covers 64 contiguous bytes of each of 16 rows and the pair of
// instructions whole 128-byte lines.  Nothing is staged in LDS and nothing
// waits on a barrier: memory latency is hidden by a one-step register
// prefetch and by several wavefronts per SIMD.  Measured on MI355X, loads of
// this shape stream HBM at the rate of fully contiguous ones (5.6 TB/s on a
// 389 MB matrix), while LDS-DMA staging needs far more bytes in flight per CU
// for the same rate.
//
// Quantisation groups.  A lane's piece is 32 consecutive k; the four pieces of
// one 64-byte half (lanes kg = 0..3) span 128 k, i.e. 2 groups at gs = 64 and
// 4 at gs = 32, while a 16x16x32 MFMA sums over all four lane groups.
// Cross-lane swaps regroup the words so that each MFMA operand register holds
// one quantisation group:
//   gs = 128: no swap; register j = word j of every lane (one group);
//   gs = 64:  swap32(w0, w2), swap32(w1, w3): registers 0, 1 = group 0
//             (lanes kg < 2 keep their words 0 / 1, lanes kg >= 2 receive
//             words 2 / 3 of lane - 32), registers 2, 3 = group 1;
//   gs = 32:  the above, then swap16(w0, w1), swap16(w2, w3): register j =
//             word kg of lane group j = group j.
// (v_permlane32_swap exchanges the upper 32 lanes of its first operand with
// the lower 32 lanes of its second; v_permlane16_swap the odd 16-lane rows of
// the first with the even rows of the second.)  The activation operand of
// MFMA slot j is loaded to match: lane (m, kg) takes the 8 k its weight lane
// holds, k = 32 g' + 8 j' (relative to the 128-k half) with
//   gs = 128: g' = kg, j' = j;
//   gs = 64:  g' = (kg & 1) + 2 (j >> 1), j' = (j & 1) + 2 (kg >> 1);
//   gs = 32:  g' = j, j' = kg.
//
// Arithmetic per tile and quantisation group g (P and the accumulators in the
// MFMA output layout, lane (n, kg) register r = [m = 4 kg + r][n]):
//   P_g = sum over the group's slots of MFMA(x, OFF + q)      (exact products)
//   acc += s_g * P_g                                          (4 FMAs per lane)
// and, per four groups, one v_mfma_f32_16x16x4_f32 adds
// sum_g X[m, g] (b_g - OFF s_g) into a second accumulator: X[m, 4 bb + kg]
// reaches lane (m, kg) from MFMAs of the activation slots against selector
// operands (A-operand rows 4g .. 4g + 3 all ones, the others zero), and lane
// (n, kg) loads the scale and bias of its own group 4 bb + kg.
#pragma once

#include "dfmi_device.h"

namespace dfmi {

constexpr int kDirectK = 256;        // k per step: 128 bytes of every int4 weight row
constexpr int kDirectMaxWaves = 8;   // wavefronts of a workgroup (they split K)

__device__ inline void swap32(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

__device__ inline void swap16(uint32_t& a, uint32_t& b) {
  const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
  a = r[0];
  b = r[1];
}

template <typename Tag, int GS, int NT>
struct Direct {
  static_assert(GS == 32 || GS == 64 || GS == 128, "group size");
  static constexpr int GPS = kDirectK / GS;        // quantisation groups per step (8, 4, 2)
  static constexpr int NBB = (GPS + 3) / 4;        // bias MFMAs per tile and step
  static constexpr int SV = GPS / 2;               // u32 registers of the step's packed scales
  static constexpr int RED_FLOATS = NT * 4 * 64;   // one wavefront's partial tiles

  struct Ctx {
    __amdgpu_buffer_rsrc_t x, w, s, b;
    uint32_t xoff;      // byte offset of this lane's activation row + its slot base
    uint32_t woff[NT];  // byte offset of this lane's weight piece in tile t (step 0)
    uint32_t soff[NT];  // byte offset of the scales of this lane's row (step 0)
    uint32_t ooff[NT];  // byte offset of this lane's own-group scale / bias (step 0)
    uint32_t omask;     // 0xFFFF, or 0 for a lane whose own group lies past the step
  };

  // HBM streams of one step, prefetched a step ahead.
  struct Step {
    u32x4 w[NT][2];           // packed words of the two 64-byte halves
    uint32_t s[NT][SV];       // the step's GPS scales of this lane's row, packed pairs
    uint32_t so[NT][NBB];     // scale of group 4 bb + kg of this lane's row
    uint32_t bo[NT][NBB];     // bias of that group
  };

  // Activations of one step (L1 / L2 resident: every wavefront of the GPU
  // reads the same x), loaded when the step's computation starts.
  struct XStep {
    u32x4 v[2][4];            // half h, MFMA slot j
  };

  // k offset (elements, within a 128-k half) of slot j for lane group kg:
  // lane part + slot part (the slot part is wave-uniform: an immediate).
  __device__ static constexpr int slot_k(int j) {
    return GS == 128 ? 8 * j : (GS == 64 ? 64 * (j >> 1) + 8 * (j & 1) : 32 * j);
  }
  __device__ static inline int lane_k(int kg) {
    return GS == 128 ? 32 * kg : (GS == 64 ? 32 * (kg & 1) + 16 * (kg >> 1) : 8 * kg);
  }
  // quantisation group (within the step) of half h, slot j
  __device__ static constexpr int group_of(int h, int j) {
    return GS == 128 ? h : (GS == 64 ? 2 * h + (j >> 1) : 4 * h + j);
  }

  __device__ static inline Ctx setup(const uint16_t* x, const uint32_t* w, const uint16_t* s,
                                     const uint16_t* b, int M, int K, int N, int n0, int lane) {
    Ctx c;
    const int col = lane & 15, kg = lane >> 4;
    const uint32_t groups = (uint32_t)(K / GS);
    c.x = buffer_rsrc(x, (uint32_t)M * (uint32_t)K * 2u);
    c.w = buffer_rsrc(w, (uint32_t)N * (uint32_t)(K / 2));
    c.s = buffer_rsrc(s, (uint32_t)N * groups * 2u);
    c.b = buffer_rsrc(b, (uint32_t)N * groups * 2u);
    const int m = min(col, M - 1);  // rows >= M repeat row M-1 and are never stored
    c.xoff = (uint32_t)m * (uint32_t)K * 2u + 2u * (uint32_t)lane_k(kg);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const uint32_t row = (uint32_t)min(n0 + 16 * t + col, N - 1);
      c.woff[t] = row * (uint32_t)(K / 2) + 16u * (uint32_t)kg;
      c.soff[t] = row * groups * 2u;
      c.ooff[t] = c.soff[t] + 2u * (uint32_t)min(kg, GPS - 1);
    }
    c.omask = kg < GPS ? 0xFFFFu : 0u;
    return c;
  }

  __device__ static inline void load(Step& S, const Ctx& c, int i) {
    const uint32_t wst = 128u * (uint32_t)i;
    const uint32_t sst = 2u * GPS * (uint32_t)i;
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int h = 0; h < 2; ++h)
        S.w[t][h] = __builtin_amdgcn_raw_buffer_load_b128(c.w, c.woff[t] + 64u * h, wst, 0);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      if constexpr (SV == 1) {
        S.s[t][0] = __builtin_amdgcn_raw_buffer_load_b32(c.s, c.soff[t], sst, 0);
      } else if constexpr (SV == 2) {
        const u32x2 v = __builtin_amdgcn_raw_buffer_load_b64(c.s, c.soff[t], sst, 0);
        S.s[t][0] = v.x;
        S.s[t][1] = v.y;
      } else {
        const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(c.s, c.soff[t], sst, 0);
        S.s[t][0] = v.x;
        S.s[t][1] = v.y;
        S.s[t][2] = v.z;
        S.s[t][3] = v.w;
      }
#pragma unroll
      for (int bb = 0; bb < NBB; ++bb) {
        S.so[t][bb] = __builtin_amdgcn_raw_buffer_load_b16(c.s, c.ooff[t] + 8u * bb, sst, 0);
        S.bo[t][bb] = __builtin_amdgcn_raw_buffer_load_b16(c.b, c.ooff[t] + 8u * bb, sst, 0);
      }
    }
  }

  __device__ static inline void load_x(XStep& X, const Ctx& c, int i) {
    const uint32_t xst = 512u * (uint32_t)i;
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        X.v[h][j] = __builtin_amdgcn_raw_buffer_load_b128(
            c.x, c.xoff + 2u * (uint32_t)(128 * h + slot_k(j)), xst, 0);
  }

  // Regroup one half's four words so that register j holds one group (above).
  __device__ static inline void regroup(u32x4& w) {
    if constexpr (GS <= 64) {
      uint32_t w0 = w.x, w1 = w.y, w2 = w.z, w3 = w.w;
      swap32(w0, w2);
      swap32(w1, w3);
      if constexpr (GS == 32) {
        swap16(w0, w1);
        swap16(w2, w3);
      }
      w = u32x4{w0, w1, w2, w3};
    }
  }

  __device__ static inline float scale(const Step& S, int t, int g) {
    return (g & 1) ? Num<Tag>::hi(S.s[t][g >> 1]) : Num<Tag>::lo(S.s[t][g >> 1]);
  }

  __device__ static inline void compute(const Step& S, const XStep& X, const Ctx& c,
                                        f32x4 (&acc)[NT], f32x4 (&accb)[NT],
                                        const u32x4 (&sel)[4], const DqConst& dq) {
    // X[m, 4 bb + kg] in every register of lane (m, kg)
    f32x4 xs[NBB];
#pragma unroll
    for (int bb = 0; bb < NBB; ++bb) xs[bb] = zero4();
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int g = group_of(h, j);
        xs[g >> 2] = Num<Tag>::mma(sel[g & 3], X.v[h][j], xs[g >> 2]);
      }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        u32x4 w = S.w[t][h];
        regroup(w);
        const u32x4 d0 = dequant_word4<Tag>(w.x, dq);
        const u32x4 d1 = dequant_word4<Tag>(w.y, dq);
        const u32x4 d2 = dequant_word4<Tag>(w.z, dq);
        const u32x4 d3 = dequant_word4<Tag>(w.w, dq);
        if constexpr (GS == 128) {
          f32x4 p = Num<Tag>::mma(X.v[h][0], d0, zero4());
          p = Num<Tag>::mma(X.v[h][1], d1, p);
          p = Num<Tag>::mma(X.v[h][2], d2, p);
          p = Num<Tag>::mma(X.v[h][3], d3, p);
          fma_acc(acc[t], scale(S, t, h), p);
        } else if constexpr (GS == 64) {
          f32x4 p0 = Num<Tag>::mma(X.v[h][0], d0, zero4());
          f32x4 p1 = Num<Tag>::mma(X.v[h][2], d2, zero4());
          p0 = Num<Tag>::mma(X.v[h][1], d1, p0);
          p1 = Num<Tag>::mma(X.v[h][3], d3, p1);
          fma_acc(acc[t], scale(S, t, 2 * h), p0);
          fma_acc(acc[t], scale(S, t, 2 * h + 1), p1);
        } else {
          const f32x4 p0 = Num<Tag>::mma(X.v[h][0], d0, zero4());
          const f32x4 p1 = Num<Tag>::mma(X.v[h][1], d1, zero4());
          const f32x4 p2 = Num<Tag>::mma(X.v[h][2], d2, zero4());
          const f32x4 p3 = Num<Tag>::mma(X.v[h][3], d3, zero4());
          fma_acc(acc[t], scale(S, t, 4 * h), p0);
          fma_acc(acc[t], scale(S, t, 4 * h + 1), p1);
          fma_acc(acc[t], scale(S, t, 4 * h + 2), p2);
          fma_acc(acc[t], scale(S, t, 4 * h + 3), p3);
        }
      }
#pragma unroll
      for (int bb = 0; bb < NBB; ++bb) {
        uint32_t so = S.so[t][bb], bo = S.bo[t][bb];
        if constexpr (GPS < 4) {
          so &= c.omask;
          bo &= c.omask;
        }
        const float bq = __builtin_fmaf(-Num<Tag>::OFF, Num<Tag>::h2f(so), Num<Tag>::h2f(bo));
        accb[t] = mma_f32_16x16x4(xs[bb].x, bq, accb[t]);
      }
    }
  }

  __device__ static inline void fma_acc(f32x4& acc, float s, const f32x4& p) {
    acc.x = __builtin_fmaf(s, p.x, acc.x);
    acc.y = __builtin_fmaf(s, p.y, acc.y);
    acc.z = __builtin_fmaf(s, p.z, acc.z);
    acc.w = __builtin_fmaf(s, p.w, acc.w);
  }

  // Selector operands: lane value ONE2 where (lane & 15) >> 2 == g.
  __device__ static inline void selectors(u32x4 (&sel)[4], int lane) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const uint32_t v = ((lane & 15) >> 2) == g ? Num<Tag>::ONE2 : 0u;
      sel[g] = u32x4{v, v, v, v};
    }
  }

  // Accumulate steps [i0, i1) (i1 > i0) into acc.  Two register sets; step
  // i+1 is in flight while step i is computed.  Loads sit in straight-line
  // code (the loop runs while both prefetches are valid, the tail is
  // peeled), so the compiler waits for exactly the older set.
  __device__ static inline void step(const Step& S, const Ctx& c, int i, f32x4 (&acc)[NT],
                                     f32x4 (&accb)[NT], const u32x4 (&sel)[4],
                                     const DqConst& dq) {
    XStep X;
    load_x(X, c, i);
    compute(S, X, c, acc, accb, sel, dq);
  }

  __device__ static inline void run(const Ctx& c, int i0, int i1, f32x4 (&acc)[NT], int lane) {
    const DqConst dq = dq_const<Tag>();
    u32x4 sel[4];
    selectors(sel, lane);
    f32x4 accb[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) accb[t] = zero4();
    Step A, B;
    if (i1 - i0 <= 2) {
      // short range: every load of the wavefront in one round trip
      XStep XA, XB;
      load(A, c, i0);
      load_x(XA, c, i0);
      if (i1 - i0 == 2) {
        load(B, c, i0 + 1);
        load_x(XB, c, i0 + 1);
      }
      __builtin_amdgcn_sched_barrier(0);
      compute(A, XA, c, acc, accb, sel, dq);
      if (i1 - i0 == 2) compute(B, XB, c, acc, accb, sel, dq);
#pragma unroll
      for (int t = 0; t < NT; ++t) acc[t] += accb[t];
      return;
    }
    load(A, c, i0);
    {
      load(B, c, i0 + 1);
      __builtin_amdgcn_sched_barrier(0);
      int i = i0;
      for (; i + 3 < i1; i += 2) {
        step(A, c, i, acc, accb, sel, dq);
        load(A, c, i + 2);
        __builtin_amdgcn_sched_barrier(0);
        step(B, c, i + 1, acc, accb, sel, dq);
        load(B, c, i + 3);
        __builtin_amdgcn_sched_barrier(0);
      }
      if (i1 - i == 3) {
        step(A, c, i, acc, accb, sel, dq);
        load(A, c, i + 2);
        __builtin_amdgcn_sched_barrier(0);
        step(B, c, i + 1, acc, accb, sel, dq);
        step(A, c, i + 2, acc, accb, sel, dq);
      } else {
        step(A, c, i, acc, accb, sel, dq);
        step(B, c, i + 1, acc, accb, sel, dq);
      }
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t] += accb[t];
  }
};

}  // namespace dfmi
