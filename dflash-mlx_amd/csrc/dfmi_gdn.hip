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
// by the whole workgroup first (one memory round trip per chunk instead of
// one per step); the dot products reduce over the 32 lanes with DPP row
// operations and one v_permlane16_swap.
// The state is fp32 across the steps of the recurrence; the replay rounds it
// to the state dtype after every unmasked step, as the reference kernel does.
#include <algorithm>

#include "dfmi_device.h"
#include "dfmi_host.h"

namespace dfmi {

constexpr int kGdnRows = 8;      // state rows per workgroup (one per 32 lanes)
constexpr int kGdnThreads = 256;
constexpr int kGdnStageFloats = 16 * 128;  // per staged key / query chunk: TC * Dk
constexpr int kGdnMaxChunk = kGdnThreads / kGdnRows;  // steps per chunk: one value per thread

__device__ inline float ld_any(const void* p, int64_t i, int dtype) {
  if (dtype == DFMI_F32) return static_cast<const float*>(p)[i];
  const uint16_t h = static_cast<const uint16_t*>(p)[i];
  return dtype == DFMI_BF16 ? Num<BF16>::h2f(h) : Num<F16>::h2f(h);
}

__device__ inline void st_any(void* p, int64_t i, int dtype, float v) {
  if (dtype == DFMI_F32) static_cast<float*>(p)[i] = v;
  else if (dtype == DFMI_BF16) static_cast<uint16_t*>(p)[i] = Num<BF16>::f2h(v);
  else static_cast<uint16_t*>(p)[i] = Num<F16>::f2h(v);
}

__device__ inline float round_any(float v, int dtype) {
  if (dtype == DFMI_BF16) return Num<BF16>::h2f(Num<BF16>::f2h(v));
  if (dtype == DFMI_F16) return Num<F16>::h2f(Num<F16>::f2h(v));
  return v;
}

// Sum over the 32 lanes of a half-wavefront, every lane getting the sum:
// DPP within each 16-lane row (quad swaps, then half-row and row mirrors),
// then v_permlane16_swap pairs the two rows of each half-wavefront.
template <int CTRL>
__device__ inline float dpp_add_t(float v) {
  return v + __int_as_float(
                 __builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
__device__ inline float sum32(float v) {
  v = dpp_add_t<0xB1>(v);   // quad_perm [1,0,3,2]
  v = dpp_add_t<0x4E>(v);   // quad_perm [2,3,0,1]
  v = dpp_add_t<0x141>(v);  // row_half_mirror
  v = dpp_add_t<0x140>(v);  // row_mirror: every lane holds its row's sum
  const auto pr = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false,
                                                   false);
  return __uint_as_float(pr[0]) + __uint_as_float(pr[1]);
}

// Stage n elements of a [T]-strided source into LDS: element e = t * W + c
// (t = e / W, c = e % W) comes from src[base + t * stride + c].  Up to
// kGdnStageFloats / kGdnThreads elements per thread, all loads issued before
// the first store.
template <int W>
__device__ inline void stage(const void* src, int dtype, int64_t base, int64_t stride, int n,
                            float* dst) {
  constexpr int PER = kGdnStageFloats / kGdnThreads;
  float r[PER];
  if (dtype == DFMI_F32) {
    const float* p = static_cast<const float*>(src);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = threadIdx.x + j * kGdnThreads;
      r[j] = e < n ? p[base + (int64_t)(e / W) * stride + e % W] : 0.f;
    }
  } else {
    const uint16_t* p = static_cast<const uint16_t*>(src);
    uint16_t h[PER];
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int e = threadIdx.x + j * kGdnThreads;
      h[j] = e < n ? p[base + (int64_t)(e / W) * stride + e % W] : (uint16_t)0;
    }
#pragma unroll
    for (int j = 0; j < PER; ++j)
      r[j] = dtype == DFMI_BF16 ? Num<BF16>::h2f(h[j]) : Num<F16>::h2f(h[j]);
  }
#pragma unroll
  for (int j = 0; j < PER; ++j) {
    const int e = threadIdx.x + j * kGdnThreads;
    if (e < n) dst[e] = r[j];
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
#pragma unroll
  for (int i = 0; i < NPT; ++i) st[i] = ld_any(p, i0 + i, dtype);
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
};

// REPLAY = false: gated_delta_tape; true: tape_replay.
template <int NPT, bool REPLAY>
__global__ __launch_bounds__(kGdnThreads) void gdn_kernel(GdnArgs a) {
  constexpr int DK = 32 * NPT;
  __shared__ float s_k[kGdnStageFloats];
  __shared__ float s_q[REPLAY ? 1 : kGdnStageFloats];
  __shared__ float s_g[kGdnStageFloats];          // per-key gates (or TC scalars)
  __shared__ float s_v[kGdnMaxChunk * kGdnRows];  // [TC][8] values or tape entries
  __shared__ float s_beta[kGdnMaxChunk];
  __shared__ int s_live[kGdnMaxChunk];

  const int bh = blockIdx.y;  // b * Hv + hv
  const int b = bh / a.Hv, hv = bh % a.Hv;
  const int hk = hv / (a.Hv / a.Hk);
  const int row = threadIdx.x >> 5, lane = threadIdx.x & 31;
  const int dv = blockIdx.x * kGdnRows + row;
  const bool have_row = dv < a.Dv;

  float st[NPT];
  const int64_t srow = ((int64_t)bh * a.Dv + dv) * DK + NPT * lane;
#pragma unroll
  for (int i = 0; i < NPT; ++i) st[i] = 0.f;
  if (have_row) load_row<NPT>(a.state_in, a.state_dtype, srow, a.state_vec != 0, st);

  for (int t0 = 0; t0 < a.T; t0 += a.tc) {
    const int nt = min(a.tc, a.T - t0);
    __syncthreads();  // the previous chunk's LDS is no longer read
    const int64_t kbase = (((int64_t)b * a.T + t0) * a.Hk + hk) * DK;
    stage<DK>(a.k, a.x_dtype, kbase, (int64_t)a.Hk * DK, nt * DK, s_k);
    if (!REPLAY) stage<DK>(a.q, a.x_dtype, kbase, (int64_t)a.Hk * DK, nt * DK, s_q);
    const int64_t hbase = ((int64_t)b * a.T + t0) * a.Hv + hv;  // [b, t0, hv] of [B, T, Hv]
    if (a.g_per_key) stage<DK>(a.g, a.g_dtype, hbase * DK, (int64_t)a.Hv * DK, nt * DK, s_g);
    // one value (or tape entry) per thread: rows of this workgroup x steps
    {
      const int e = threadIdx.x;  // nt * kGdnRows <= kGdnThreads
      const int t = e / kGdnRows, r = e % kGdnRows;
      const int d = blockIdx.x * kGdnRows + r;
      if (t < nt) {
        const int64_t vi = (hbase + (int64_t)t * a.Hv) * a.Dv + d;
        float val = 0.f;
        if (d < a.Dv) val = REPLAY ? a.tape_in[vi] : ld_any(a.v, vi, a.x_dtype);
        s_v[e] = val;
      }
      if (e < nt) {
        const int64_t hi = hbase + (int64_t)e * a.Hv;
        if (!a.g_per_key) s_g[e] = ld_any(a.g, hi, a.g_dtype);
        if (!REPLAY) s_beta[e] = ld_any(a.beta, hi, a.beta_dtype);
        s_live[e] = a.mask ? (a.mask[(int64_t)b * a.T + t0 + e] != 0) : 1;
      }
    }
    __syncthreads();
    for (int t = 0; t < nt; ++t) {
      const float* kt = s_k + t * DK + NPT * lane;
      const float* gt = s_g + (a.g_per_key ? t * DK + NPT * lane : t);
      const int64_t oi = (((int64_t)b * a.T + t0 + t) * a.Hv + hv) * a.Dv + dv;
      if (!s_live[t]) {  // uniform: the state stays, tape and output are zero
        if (!REPLAY && have_row && lane == 0) {
          a.tape_out[oi] = 0.f;
          st_any(a.y, oi, a.x_dtype, 0.f);
        }
        continue;
      }
#pragma unroll
      for (int i = 0; i < NPT; ++i) st[i] *= a.g_per_key ? gt[i] : gt[0];
      if (REPLAY) {
        const float d = s_v[t * kGdnRows + row];
#pragma unroll
        for (int i = 0; i < NPT; ++i) st[i] = round_any(st[i] + kt[i] * d, a.state_dtype);
      } else {
        float kv = 0.f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) kv += st[i] * kt[i];
        kv = sum32(kv);
        const float d = (s_v[t * kGdnRows + row] - kv) * s_beta[t];
        const float* qt = s_q + t * DK + NPT * lane;
        float o = 0.f;
#pragma unroll
        for (int i = 0; i < NPT; ++i) {
          st[i] += kt[i] * d;
          o += st[i] * qt[i];
        }
        o = sum32(o);
        if (have_row && lane == 0) {
          a.tape_out[oi] = d;
          st_any(a.y, oi, a.x_dtype, o);
        }
      }
    }
  }
  if (have_row) store_row<NPT>(a.state_out, a.state_dtype, srow, a.state_vec != 0, st);
}

template <bool REPLAY>
static void launch_gdn(const GdnArgs& a, hipStream_t st) {
  const dim3 grid((unsigned)((a.Dv + kGdnRows - 1) / kGdnRows), (unsigned)(a.B * a.Hv));
  switch (a.Dk / 32) {
    case 1: hipLaunchKernelGGL((gdn_kernel<1, REPLAY>), grid, dim3(kGdnThreads), 0, st, a); break;
    case 2: hipLaunchKernelGGL((gdn_kernel<2, REPLAY>), grid, dim3(kGdnThreads), 0, st, a); break;
    case 4: hipLaunchKernelGGL((gdn_kernel<4, REPLAY>), grid, dim3(kGdnThreads), 0, st, a); break;
    case 8: hipLaunchKernelGGL((gdn_kernel<8, REPLAY>), grid, dim3(kGdnThreads), 0, st, a); break;
    default: hipLaunchKernelGGL((gdn_kernel<16, REPLAY>), grid, dim3(kGdnThreads), 0, st, a); break;
  }
}

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
  a.tc = std::min(kGdnStageFloats / (int)Dk, kGdnMaxChunk);
  a.state_vec = gdn_state_vec(state_in, state_out, state_dtype);
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
  a.tc = std::min(kGdnStageFloats / (int)Dk, kGdnMaxChunk);
  a.state_vec = gdn_state_vec(state_in, state_out, state_dtype);
  launch_gdn<true>(a, static_cast<hipStream_t>(stream));
  return check_launch("dfmi_tape_replay");
}
