// GDN rollback pair on gfx950: the gated-delta recurrence that records the
// innovation tape, and the replay of that tape over the accepted steps.
//
// Both are short sequential recurrences (T steps, T = the verify block) over
// independent state rows [b, hv, dv, 0..Dk): per step a row needs the step's
// key (and query) vector of its key head, one gate, one beta and one value.
// A workgroup of 256 threads takes 8 consecutive rows of one (b, hv); each
// row is a 32-lane half-wavefront, lane j holding elements NPT j .. NPT j +
// NPT - 1 (NPT = Dk / 32) in registers for all T steps, so the state is read
// and written once.  The step inputs of a chunk of TC steps are staged in LDS
// by the whole workgroup first (every load issued before the first
// conversion: one memory round trip per chunk), with k . q of each step; the
// loop reads step t + 1's inputs from LDS while step t computes, its two dot
// products reduce over the 32 lanes with DPP row operations and one
// v_permlane16_swap, and the per-step tape entries and outputs go to LDS and
// leave in one store per chunk.
// The state is fp32 across the steps of the recurrence; the replay rounds it
// to the state dtype after every unmasked step, as the reference kernel does.
#include <algorithm>

#include "dfmi_device.h"
#include "dfmi_host.h"

namespace dfmi {

constexpr int kGdnRows = 8;      // state rows per workgroup (one per 32 lanes)
constexpr int kGdnThreads = 256;
constexpr int kGdnPer = 8;       // elements per thread of a staged key / query / gate chunk
constexpr int kGdnStageFloats = kGdnThreads * kGdnPer;  // per staged chunk: TC * Dk
constexpr int kGdnMaxChunk = 32;  // steps per chunk: one live-mask bit each
// Steps staged per chunk: the key / query / gate chunk fits a stage (TC x 8
// rows <= 256 threads holds for every TC <= 32: one (step, row) value per
// thread).
constexpr int gdn_chunk_steps(int dk) { return std::min(kGdnStageFloats / dk, kGdnMaxChunk); }

// How the replay rounds its state after every step (the state dtype); the
// recurrence keeps fp32 throughout.
constexpr int kRoundNone = 0, kRoundBF16 = 1, kRoundF16 = 2;

template <int R>
__device__ inline float round_state(float v) {
  if constexpr (R == kRoundBF16) return Num<BF16>::h2f(Num<BF16>::f2h(v));
  else if constexpr (R == kRoundF16) return Num<F16>::h2f(Num<F16>::f2h(v));
  else return v;
}

// One element in its storage form (fp32 bits or a 16-bit value): the load
// alone, so that all of a thread's loads are issued before the first
// conversion waits for one.
__device__ inline uint32_t ld_raw(const void* p, int64_t i, int dtype) {
  return dtype == DFMI_F32 ? static_cast<const uint32_t*>(p)[i]
                           : (uint32_t) static_cast<const uint16_t*>(p)[i];
}
__device__ inline float cvt_raw(uint32_t r, int dtype) {
  if (dtype == DFMI_F32) return __uint_as_float(r);
  return dtype == DFMI_BF16 ? Num<BF16>::h2f(r & 0xFFFFu) : Num<F16>::h2f(r);
}

__device__ inline void st_any(void* p, int64_t i, int dtype, float v) {
  if (dtype == DFMI_F32) static_cast<float*>(p)[i] = v;
  else if (dtype == DFMI_BF16) static_cast<uint16_t*>(p)[i] = Num<BF16>::f2h(v);
  else static_cast<uint16_t*>(p)[i] = Num<F16>::f2h(v);
}

// Sums over the 32 lanes of a half-wavefront (a state row), every lane
// getting the sum: DPP within each 16-lane row (quad swaps, then half-row and
// row mirrors), then v_permlane16_swap pairs the two rows of the
// half-wavefront.  Two independent sums go through the steps together, so
// their latencies overlap.
template <int CTRL>
__device__ inline float dpp_add_t(float v) {
  return v + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ inline float swap16_add(float v) {
  const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                   false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}
__device__ inline float swap32_add(float v) {
  const auto pr = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                   false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}
// Sum over aligned groups of G consecutive lanes (G = 2 .. 64), every lane
// getting its group's sum.
template <int G>
__device__ inline float group_sum(float v) {
  if constexpr (G >= 2) v = dpp_add_t<0xB1>(v);
  if constexpr (G >= 4) v = dpp_add_t<0x4E>(v);
  if constexpr (G >= 8) v = dpp_add_t<0x141>(v);
  if constexpr (G >= 16) v = dpp_add_t<0x140>(v);
  if constexpr (G >= 32) v = swap16_add(v);
  if constexpr (G >= 64) v = swap32_add(v);
  return v;
}
__device__ inline void sum32x2(float& a, float& b) {
  a = dpp_add_t<0xB1>(a);   // quad_perm [1,0,3,2]
  b = dpp_add_t<0xB1>(b);
  a = dpp_add_t<0x4E>(a);   // quad_perm [2,3,0,1]
  b = dpp_add_t<0x4E>(b);
  a = dpp_add_t<0x141>(a);  // row_half_mirror
  b = dpp_add_t<0x141>(b);
  a = dpp_add_t<0x140>(a);  // row_mirror: every lane holds its row's sum
  b = dpp_add_t<0x140>(b);
  a = swap16_add(a);
  b = swap16_add(b);
}

// A thread's kGdnPer consecutive elements of a staged [nt][DK] chunk (step t
// from src[base + t * stride ...]), in storage form: 16-byte vector loads when
// vec (16-byte aligned source: every piece starts at a multiple of 8
// elements), element loads otherwise; zero past step nt.
struct Raw8 {
  u32x4 a, b;  // fp32: eight values; 16-bit: a holds eight, b is unused
};

template <int DK>
__device__ inline Raw8 chunk_load(const void* src, int dtype, bool vec, int64_t base,
                                  int64_t stride, int nt) {
  Raw8 r;
  r.a = u32x4{0u, 0u, 0u, 0u};
  r.b = r.a;
  const int e0 = threadIdx.x * kGdnPer;
  const int t = e0 / DK, c = e0 % DK;
  if (t < nt) {
    const int64_t i0 = base + (int64_t)t * stride + c;
    if (dtype == DFMI_F32) {
      const uint32_t* p = static_cast<const uint32_t*>(src) + i0;
      if (vec) {
        r.a = *reinterpret_cast<const u32x4*>(p);
        r.b = *reinterpret_cast<const u32x4*>(p + 4);
      } else {
        r.a = u32x4{p[0], p[1], p[2], p[3]};
        r.b = u32x4{p[4], p[5], p[6], p[7]};
      }
    } else {
      const uint16_t* p = static_cast<const uint16_t*>(src) + i0;
      if (vec) {
        r.a = *reinterpret_cast<const u32x4*>(p);
      } else {
        r.a = u32x4{p[0] | (uint32_t)p[1] << 16, p[2] | (uint32_t)p[3] << 16,
                    p[4] | (uint32_t)p[5] << 16, p[6] | (uint32_t)p[7] << 16};
      }
    }
  }
  return r;
}

// The eight elements as floats (lo, hi), also written to dst (16-byte aligned).
__device__ inline void chunk_store(const Raw8& r, int dtype, float* dst, f32x4& lo, f32x4& hi) {
  if (dtype == DFMI_F32) {
    lo = __builtin_bit_cast(f32x4, r.a);
    hi = __builtin_bit_cast(f32x4, r.b);
  } else if (dtype == DFMI_BF16) {
    lo = f32x4{Num<BF16>::lo(r.a.x), Num<BF16>::hi(r.a.x), Num<BF16>::lo(r.a.y),
               Num<BF16>::hi(r.a.y)};
    hi = f32x4{Num<BF16>::lo(r.a.z), Num<BF16>::hi(r.a.z), Num<BF16>::lo(r.a.w),
               Num<BF16>::hi(r.a.w)};
  } else {
    lo = f32x4{Num<F16>::lo(r.a.x), Num<F16>::hi(r.a.x), Num<F16>::lo(r.a.y),
               Num<F16>::hi(r.a.y)};
    hi = f32x4{Num<F16>::lo(r.a.z), Num<F16>::hi(r.a.z), Num<F16>::lo(r.a.w),
               Num<F16>::hi(r.a.w)};
  }
  *reinterpret_cast<f32x4*>(dst) = lo;
  *reinterpret_cast<f32x4*>(dst + 4) = hi;
}

// NPT floats of one LDS row piece (16-byte aligned when NPT % 4 == 0).
template <int NPT>
__device__ inline void lds_piece(const float* p, float (&r)[NPT]) {
  if constexpr (NPT % 4 == 0) {
#pragma unroll
    for (int i = 0; i < NPT; i += 4) {
      const f32x4 v = *reinterpret_cast<const f32x4*>(p + i);
      r[i] = v.x;
      r[i + 1] = v.y;
      r[i + 2] = v.z;
      r[i + 3] = v.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < NPT; ++i) r[i] = p[i];
  }
}

// A lane's NPT consecutive state elements: 16-byte vector accesses when the
// row pieces are aligned (NPT % 4 == 0 and vec), element accesses otherwise.
template <int NPT>
__device__ inline void load_row(const void* p, int dtype, int64_t i0, bool vec, float (&st)[NPT]) {
  if constexpr (NPT % 4 == 0) {
    if (vec && dtype == DFMI_F32) {
#pragma unroll
      for (int i = 0; i < NPT; i += 4) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(static_cast<const float*>(p) + i0 + i);
        st[i] = v[0];
        st[i + 1] = v[1];
        st[i + 2] = v[2];
        st[i + 3] = v[3];
      }
      return;
    }
    if (vec) {
#pragma unroll
      for (int i = 0; i < NPT; i += 4) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(static_cast<const uint16_t*>(p) + i0 + i);
        const bool bf = dtype == DFMI_BF16;
        st[i] = bf ? Num<BF16>::lo(v.x) : Num<F16>::lo(v.x);
        st[i + 1] = bf ? Num<BF16>::hi(v.x) : Num<F16>::hi(v.x);
        st[i + 2] = bf ? Num<BF16>::lo(v.y) : Num<F16>::lo(v.y);
        st[i + 3] = bf ? Num<BF16>::hi(v.y) : Num<F16>::hi(v.y);
      }
      return;
    }
  }
  uint32_t r[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) r[i] = ld_raw(p, i0 + i, dtype);
#pragma unroll
  for (int i = 0; i < NPT; ++i) st[i] = cvt_raw(r[i], dtype);
}

template <int NPT>
__device__ inline void store_row(void* p, int dtype, int64_t i0, bool vec, const float (&st)[NPT]) {
  if constexpr (NPT % 4 == 0) {
    if (vec && dtype == DFMI_F32) {
#pragma unroll
      for (int i = 0; i < NPT; i += 4)
        *reinterpret_cast<f32x4*>(static_cast<float*>(p) + i0 + i) =
            f32x4{st[i], st[i + 1], st[i + 2], st[i + 3]};
      return;
    }
    if (vec) {
      const bool bf = dtype == DFMI_BF16;
#pragma unroll
      for (int i = 0; i < NPT; i += 4) {
        uint32_t h[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) h[j] = bf ? Num<BF16>::f2h(st[i + j]) : Num<F16>::f2h(st[i + j]);
        *reinterpret_cast<u32x2*>(static_cast<uint16_t*>(p) + i0 + i) =
            u32x2{h[0] | (h[1] << 16), h[2] | (h[3] << 16)};
      }
      return;
    }
  }
#pragma unroll
  for (int i = 0; i < NPT; ++i) st_any(p, i0 + i, dtype, st[i]);
}

struct GdnArgs {
  const void* q;      // [B, T, Hk, Dk]    (tape kernel only)
  const void* k;      // [B, T, Hk, Dk]
  const void* v;      // [B, T, Hv, Dv]    (tape kernel only)
  const void* g;      // [B, T, Hv] or [B, T, Hv, Dk]
  const void* beta;   // [B, T, Hv]        (tape kernel only)
  const float* tape_in;  // [B, T, Hv, Dv] (replay only)
  const void* state_in;  // [B, Hv, Dv, Dk]
  const uint8_t* mask;   // [B, T] or null
  void* y;               // [B, T, Hv, Dv] (tape kernel only)
  void* state_out;       // [B, Hv, Dv, Dk]
  float* tape_out;       // [B, T, Hv, Dv] (tape kernel only)
  int B, T, Hk, Hv, Dk, Dv;
  int x_dtype, g_dtype, beta_dtype, state_dtype;  // x: q / k / v / y (tape kernel); k (replay)
  int g_per_key;
  int tc;         // steps staged per chunk
  int state_vec;  // state_in / state_out 16-byte (fp32) or 8-byte (16-bit) aligned
  int kq_vec;     // k (and q) 16-byte aligned
  int g_vec;      // per-key g 16-byte aligned
};

// Step inputs of one step, read from LDS one step ahead of their use.
template <int NPT>
struct GdnStep {
  float k[NPT], q[NPT], g[NPT];
  float v, beta;  // value (replay: tape entry), beta
  float kq;       // k . q of the step
};

// REPLAY = false: gated_delta_tape; true: tape_replay (state rounded by RND
// after every step).  NPT = Dk / 32 state elements per lane.
template <int NPT, bool REPLAY, int RND>
__global__ __launch_bounds__(kGdnThreads) void gdn_kernel(GdnArgs a) {
  constexpr int DK = 32 * NPT;
  constexpr int RPW = kGdnRows;
  __shared__ __attribute__((aligned(16))) float s_k[kGdnStageFloats];
  __shared__ __attribute__((aligned(16))) float s_q[REPLAY ? 4 : kGdnStageFloats];
  __shared__ __attribute__((aligned(16))) float s_g[kGdnStageFloats];  // gates, per key
  __shared__ float s_v[kGdnThreads];  // [TC][RPW] values or tape entries
  __shared__ float s_beta[kGdnMaxChunk];
  __shared__ float s_kq[kGdnMaxChunk];  // k . q of every step (one key head per workgroup)
  __shared__ float s_y[REPLAY ? 1 : kGdnThreads];  // [TC][RPW] outputs
  __shared__ float s_d[REPLAY ? 1 : kGdnThreads];  // [TC][RPW] innovations
  __shared__ uint32_t s_live;                                  // bit t: step t unmasked

  const int bh = blockIdx.y;  // b * Hv + hv
  const int b = bh / a.Hv, hv = bh % a.Hv;
  const int hk = hv / (a.Hv / a.Hk);
  const int tid = threadIdx.x;
  const int row = tid >> 5, lane = tid & 31;
  const int dv = blockIdx.x * RPW + row;
  const bool have_row = dv < a.Dv;
  // this thread's (step, row) for the per-step values and outputs
  const int vt = tid / RPW, vr = tid % RPW;
  const int vd = blockIdx.x * RPW + vr;

  float st[NPT];
  const int64_t srow = ((int64_t)bh * a.Dv + dv) * DK + NPT * lane;
#pragma unroll
  for (int i = 0; i < NPT; ++i) st[i] = 0.f;
  if (have_row) load_row<NPT>(a.state_in, a.state_dtype, srow, a.state_vec != 0, st);

  for (int t0 = 0; t0 < a.T; t0 += a.tc) {
    const int nt = min(a.tc, a.T - t0);
    __syncthreads();  // the previous chunk's LDS is no longer read
    // every load of the chunk's step inputs, then the conversions into LDS
    const int64_t kbase = (((int64_t)b * a.T + t0) * a.Hk + hk) * DK;
    const int64_t kstride = (int64_t)a.Hk * DK;
    const int64_t hbase = ((int64_t)b * a.T + t0) * a.Hv + hv;  // [b, t0, hv] of [B, T, Hv]
    const Raw8 rk = chunk_load<DK>(a.k, a.x_dtype, a.kq_vec != 0, kbase, kstride, nt);
    Raw8 rq = rk;
    if constexpr (!REPLAY) rq = chunk_load<DK>(a.q, a.x_dtype, a.kq_vec != 0, kbase, kstride, nt);
    Raw8 rg = rk;
    uint32_t rgs = 0;
    const int tg = tid * kGdnPer / DK;  // step of this thread's gate piece
    if (a.g_per_key)
      rg = chunk_load<DK>(a.g, a.g_dtype, a.g_vec != 0, hbase * DK, (int64_t)a.Hv * DK, nt);
    else if (tg < nt)
      rgs = ld_raw(a.g, hbase + (int64_t)tg * a.Hv, a.g_dtype);
    uint32_t rv = 0, rb = 0;
    bool live = false;
    if (vt < nt && vd < a.Dv) {
      const int64_t vi = (hbase + (int64_t)vt * a.Hv) * a.Dv + vd;
      rv = REPLAY ? __float_as_uint(a.tape_in[vi]) : ld_raw(a.v, vi, a.x_dtype);
    }
    if (tid < nt) {
      if (!REPLAY) rb = ld_raw(a.beta, hbase + (int64_t)tid * a.Hv, a.beta_dtype);
      live = a.mask ? a.mask[(int64_t)b * a.T + t0 + tid] != 0 : true;
    }
    f32x4 klo, khi;
    chunk_store(rk, a.x_dtype, s_k + tid * kGdnPer, klo, khi);
    if constexpr (!REPLAY) {
      // k . q of step tg from the pieces this thread holds: the DK / 8
      // threads of a step are consecutive lanes of one wavefront
      f32x4 qlo, qhi;
      chunk_store(rq, a.x_dtype, s_q + tid * kGdnPer, qlo, qhi);
      float p = klo.x * qlo.x;
      p += klo.y * qlo.y;
      p += klo.z * qlo.z;
      p += klo.w * qlo.w;
      p += khi.x * qhi.x;
      p += khi.y * qhi.y;
      p += khi.z * qhi.z;
      p += khi.w * qhi.w;
      p = group_sum<DK / kGdnPer>(p);
      if (tid % (DK / kGdnPer) == 0 && tg < nt) s_kq[tg] = p;
    }
    if (a.g_per_key) {
      f32x4 glo, ghi;
      chunk_store(rg, a.g_dtype, s_g + tid * kGdnPer, glo, ghi);
    } else {  // the step's scalar gate, repeated over the key dimension
      const float gv = cvt_raw(rgs, a.g_dtype);
      *reinterpret_cast<f32x4*>(s_g + tid * kGdnPer) = f32x4{gv, gv, gv, gv};
      *reinterpret_cast<f32x4*>(s_g + tid * kGdnPer + 4) = f32x4{gv, gv, gv, gv};
    }
    if (vt < nt) s_v[tid] = REPLAY ? __uint_as_float(rv) : cvt_raw(rv, a.x_dtype);
    if (!REPLAY && tid < nt) s_beta[tid] = cvt_raw(rb, a.beta_dtype);
    if (tid < 64) {  // steps 0 .. nt-1 belong to wavefront 0
      const uint64_t bal = __ballot(live);
      if (tid == 0) s_live = (uint32_t)bal;
    }
    __syncthreads();
    const uint32_t live_bits = __builtin_amdgcn_readfirstlane(s_live);

    auto fetch = [&](GdnStep<NPT>& in, int t) {
      lds_piece<NPT>(s_k + t * DK + NPT * lane, in.k);
      lds_piece<NPT>(s_g + t * DK + NPT * lane, in.g);
      if constexpr (!REPLAY) {
        lds_piece<NPT>(s_q + t * DK + NPT * lane, in.q);
        in.beta = s_beta[t];
        in.kq = s_kq[t];
      }
      in.v = s_v[t * RPW + row];
    };
    auto advance = [&](const GdnStep<NPT>& in, int t) {
      const bool on = (live_bits >> t) & 1u;  // uniform
      if constexpr (REPLAY) {
        if (on) {
#pragma unroll
          for (int i = 0; i < NPT; ++i) {
            st[i] *= in.g[i];
            st[i] = round_state<RND>(st[i] + in.k[i] * in.v);
          }
        }
      } else {
        float d = 0.f, o = 0.f;  // a masked step leaves the state; tape and output are zero
        if (on) {
          // kv = S'.k and S'.q over the decayed state S'; then
          // y = (S' + d k^T).q = S'.q + d (k.q), so both sums share one
          // reduction and k.q comes from the staging
          float kv = 0.f, sq = 0.f;
#pragma unroll
          for (int i = 0; i < NPT; ++i) {
            st[i] *= in.g[i];
            kv += st[i] * in.k[i];
            sq += st[i] * in.q[i];
          }
          sum32x2(kv, sq);
          d = (in.v - kv) * in.beta;
#pragma unroll
          for (int i = 0; i < NPT; ++i) st[i] += in.k[i] * d;
          o = sq + d * in.kq;
        }
        if (lane == 0) {
          s_d[t * RPW + row] = d;
          s_y[t * RPW + row] = o;
        }
      }
    };
    // two register sets: the LDS reads of step t + 1 are issued before step
    // t is computed
    GdnStep<NPT> A, B;
    fetch(A, 0);
    // step 0's reads complete before the loop: otherwise the wait the
    // compiler places for them at the loop head also waits, on every step,
    // for the reads of the following step
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0); vmcnt, expcnt untouched
    for (int t = 0; t < nt; t += 2) {
      if (t + 1 < nt) fetch(B, t + 1);
      advance(A, t);
      if (t + 1 >= nt) break;
      if (t + 2 < nt) fetch(A, t + 2);
      advance(B, t + 1);
    }
    if constexpr (!REPLAY) {
      __syncthreads();
      // the chunk's tape entries and outputs: thread -> (step vt, row vr)
      if (vt < nt && vd < a.Dv) {
        const int64_t oi = (hbase + (int64_t)vt * a.Hv) * a.Dv + vd;
        a.tape_out[oi] = s_d[tid];
        st_any(a.y, oi, a.x_dtype, s_y[tid]);
      }
    }
  }
  if (have_row) store_row<NPT>(a.state_out, a.state_dtype, srow, a.state_vec != 0, st);
}

template <int NPT>
static void launch_gdn_npt(const GdnArgs& a, bool replay, hipStream_t st) {
  const dim3 grid((unsigned)((a.Dv + kGdnRows - 1) / kGdnRows), (unsigned)(a.B * a.Hv));
  const dim3 blk(kGdnThreads);
  if (!replay)
    hipLaunchKernelGGL((gdn_kernel<NPT, false, kRoundNone>), grid, blk, 0, st, a);
  else if (a.state_dtype == DFMI_BF16)
    hipLaunchKernelGGL((gdn_kernel<NPT, true, kRoundBF16>), grid, blk, 0, st, a);
  else if (a.state_dtype == DFMI_F16)
    hipLaunchKernelGGL((gdn_kernel<NPT, true, kRoundF16>), grid, blk, 0, st, a);
  else
    hipLaunchKernelGGL((gdn_kernel<NPT, true, kRoundNone>), grid, blk, 0, st, a);
}

template <bool REPLAY>
static void launch_gdn(const GdnArgs& a, hipStream_t st) {
  switch (a.Dk / 32) {
    case 1: launch_gdn_npt<1>(a, REPLAY, st); break;
    case 2: launch_gdn_npt<2>(a, REPLAY, st); break;
    case 4: launch_gdn_npt<4>(a, REPLAY, st); break;
    case 8: launch_gdn_npt<8>(a, REPLAY, st); break;
    default: launch_gdn_npt<16>(a, REPLAY, st); break;
  }
}

static bool aligned16p(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

static int gdn_state_vec(const void* in, const void* out, int dtype) {
  const uintptr_t al = dtype == DFMI_F32 ? 16 : 8;
  return (reinterpret_cast<uintptr_t>(in) % al == 0 && reinterpret_cast<uintptr_t>(out) % al == 0)
             ? 1
             : 0;
}

static bool gdn_dtype_ok(int d) { return d == DFMI_BF16 || d == DFMI_F16 || d == DFMI_F32; }

static int gdn_validate(const char* fn, int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk,
                        int64_t Dv, int x_dtype, int g_dtype, int beta_dtype, int state_dtype) {
  if (!gdn_dtype_ok(x_dtype) || !gdn_dtype_ok(g_dtype) || !gdn_dtype_ok(beta_dtype) ||
      !gdn_dtype_ok(state_dtype)) {
    set_error("%s: dtypes must be bf16, f16 or f32", fn);
    return DFMI_EINVAL;
  }
  const int64_t npt = Dk / 32;
  if (B < 0 || T < 0 || Hk < 1 || Hv < 1 || Dv < 0 || Hv % Hk != 0 || Dk % 32 != 0 ||
      !(npt == 1 || npt == 2 || npt == 4 || npt == 8 || npt == 16) || B * Hv > 65535 ||
      B * T * Hv * std::max(Dv, Dk) >= (1ll << 40)) {
    set_error("%s: unsupported shape B=%lld T=%lld Hk=%lld Hv=%lld Dk=%lld Dv=%lld (Dk in "
              "{32,64,128,256,512}, Hv a multiple of Hk)",
              fn, (long long)B, (long long)T, (long long)Hk, (long long)Hv, (long long)Dk,
              (long long)Dv);
    return DFMI_EINVAL;
  }
  return DFMI_OK;
}

}  // namespace dfmi

using namespace dfmi;

extern "C" int dfmi_gated_delta_tape(const void* q, const void* k, const void* v, const void* g,
                                     const void* beta, const void* state_in, const uint8_t* mask,
                                     void* y, void* state_out, float* tape, int64_t B, int64_t T,
                                     int64_t Hk, int64_t Hv, int64_t Dk, int64_t Dv,
                                     int qkv_dtype, int g_dtype, int beta_dtype, int state_dtype,
                                     int g_per_key, void* stream) {
  int rc = gdn_validate("dfmi_gated_delta_tape", B, T, Hk, Hv, Dk, Dv, qkv_dtype, g_dtype,
                        beta_dtype, state_dtype);
  if (rc != DFMI_OK) return rc;
  if (B == 0 || Dv == 0) return DFMI_OK;
  if (!q || !k || !v || !g || !beta || !state_in || !state_out || (T > 0 && (!y || !tape))) {
    set_error("dfmi_gated_delta_tape: null pointer");
    return DFMI_EINVAL;
  }
  GdnArgs a{};
  a.q = q;
  a.k = k;
  a.v = v;
  a.g = g;
  a.beta = beta;
  a.state_in = state_in;
  a.mask = mask;
  a.y = y;
  a.state_out = state_out;
  a.tape_out = tape;
  a.B = (int)B;
  a.T = (int)T;
  a.Hk = (int)Hk;
  a.Hv = (int)Hv;
  a.Dk = (int)Dk;
  a.Dv = (int)Dv;
  a.x_dtype = qkv_dtype;
  a.g_dtype = g_dtype;
  a.beta_dtype = beta_dtype;
  a.state_dtype = state_dtype;
  a.g_per_key = g_per_key ? 1 : 0;
  a.tc = gdn_chunk_steps((int)Dk);
  a.state_vec = gdn_state_vec(state_in, state_out, state_dtype);
  a.kq_vec = aligned16p(k) && aligned16p(q);
  a.g_vec = g_per_key && aligned16p(g);
  launch_gdn<false>(a, static_cast<hipStream_t>(stream));
  return check_launch("dfmi_gated_delta_tape");
}

extern "C" int dfmi_tape_replay(const float* tape, const void* k, const void* g,
                                const void* state_in, const uint8_t* mask, void* state_out,
                                int64_t B, int64_t T, int64_t Hk, int64_t Hv, int64_t Dk,
                                int64_t Dv, int k_dtype, int g_dtype, int state_dtype,
                                int g_per_key, void* stream) {
  int rc = gdn_validate("dfmi_tape_replay", B, T, Hk, Hv, Dk, Dv, k_dtype, g_dtype, DFMI_F32,
                        state_dtype);
  if (rc != DFMI_OK) return rc;
  if (B == 0 || Dv == 0) return DFMI_OK;
  if (!k || !g || !state_in || !state_out || (T > 0 && !tape)) {
    set_error("dfmi_tape_replay: null pointer");
    return DFMI_EINVAL;
  }
  GdnArgs a{};
  a.k = k;
  a.g = g;
  a.tape_in = tape;
  a.state_in = state_in;
  a.mask = mask;
  a.state_out = state_out;
  a.B = (int)B;
  a.T = (int)T;
  a.Hk = (int)Hk;
  a.Hv = (int)Hv;
  a.Dk = (int)Dk;
  a.Dv = (int)Dv;
  a.x_dtype = k_dtype;
  a.g_dtype = g_dtype;
  a.beta_dtype = DFMI_F32;
  a.state_dtype = state_dtype;
  a.g_per_key = g_per_key ? 1 : 0;
  a.tc = gdn_chunk_steps((int)Dk);
  a.state_vec = gdn_state_vec(state_in, state_out, state_dtype);
  a.kq_vec = aligned16p(k);
  a.g_vec = g_per_key && aligned16p(g);
  launch_gdn<true>(a, static_cast<hipStream_t>(stream));
  return check_launch("dfmi_tape_replay");
}
