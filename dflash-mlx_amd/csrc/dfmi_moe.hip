// Routed-expert (MoE) matmuls on gfx950: gather_qmm, the fused SwiGLU front
// half of a SwitchGLU block, and the weighted top-k combine.
//
// Pairs p < P map (activation row lhs_rows[p], expert rhs_experts[p]).  A run
// is a maximal stretch of consecutive pairs with the same expert (after the
// sort mlx-lm's SwitchGLU applies for >= 64 pairs, every expert is one run;
// unsorted pairs just make shorter runs).  Grid: (column blocks, P); the
// workgroup of the first pair of a run streams that expert's weight rows once
// for the whole run, 16 gathered activation rows per MFMA block, and the
// other pairs' workgroups exit at once.
//
//  * gather_stream_kernel (K >= 1024, a multiple of 256 and of 8 groups): the
//    streaming main loop (LDS-DMA staging of whole weight lines, 4
//    wavefronts) over a 64-row block: 64 rows of one expert, or for the fused
//    SwiGLU 32 gate rows and the same 32 up rows, so one workgroup produces
//    32 finished h columns.  The activation DMA takes its rows from lhs_rows.
//  * gather_kernel (every other shape): the general main loop (Core:
//    wavefronts split K, partial tiles summed through LDS), with the
//    activation row of each MFMA lane taken from lhs_rows.
#include <algorithm>
#include <cmath>

#include "dfmi_core.h"
#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

struct GatherArgs {
  const uint16_t* x;
  int64_t x_rows;
  const uint32_t* w[2];  // [0]: the matmul's (or gate) weights, [1]: up weights (SwiGLU)
  const uint16_t* s[2];
  const uint16_t* b[2];
  const int32_t* lhs;    // NULL: row p for pair p
  const int32_t* rhs;
  uint16_t* y;           // [P, N]
  int P, K, N, E;
  int chunks;
};

template <typename Tag>
__device__ inline float rnd(float v) {
  return Num<Tag>::h2f(Num<Tag>::f2h(v));
}

// silu(g) * u with every op rounded to the activation dtype, as the
// op-by-op MLX sequence sigmoid(g) -> g * sig -> * u does.
template <typename Tag>
__device__ inline float silu_mul(float g, float u) {
  const float sig = rnd<Tag>(1.0f / (1.0f + __expf(-g)));
  const float si = rnd<Tag>(g * sig);
  return si * u;
}

template <typename Tag, int GS, int NT, bool KFULL, bool GLU>
__global__ __launch_bounds__(kMaxWaves * 64) void gather_kernel(GatherArgs a) {
  constexpr int TT = GLU ? 2 * NT : NT;  // Core tiles: the NT gate tiles, then NT up tiles
  using C = Core<Tag, GS, 1, TT, KFULL>;
  __shared__ __attribute__((aligned(16))) float lds[C::LDS_BYTES / 4];

  const int p = blockIdx.y;
  const int e = a.rhs[p];
  if (p > 0 && a.rhs[p - 1] == e) return;  // not the first pair of its run (uniform)
  int run = 1;
  while (p + run < a.P && a.rhs[p + run] == e) ++run;

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  const bool bad_e = e < 0 || e >= a.E;
  const int ee = bad_e ? 0 : e;
  const uint32_t kw = (uint32_t)(a.K / 8);
  const uint32_t kgrp = (uint32_t)(a.K / GS);

  typename C::Rows r;
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int which = (GLU && t >= NT) ? 1 : 0;
    const int tt = t % NT;
    const int row = min(n0 + tt * 16 + (lane & 15), a.N - 1);
    r.wbase[t] = a.w[which] + (size_t)ee * a.N * kw;
    r.sbase[t] = a.s[which] + (size_t)ee * a.N * kgrp;
    r.bbase[t] = a.b[which] + (size_t)ee * a.N * kgrp;
    r.woff[t] = (uint32_t)row * kw;
    r.soff[t] = (uint32_t)row * kgrp;
  }

  for (int g0 = 0; g0 < run; g0 += 16) {
    const int rows = min(16, run - g0);
    // activation row of this lane's MFMA row (rows past the run repeat the last pair)
    const int pl = p + g0 + min(lane & 15, rows - 1);
    int xr_row = a.lhs ? a.lhs[pl] : pl;
    if (xr_row < 0 || xr_row >= a.x_rows) xr_row = 0;  // reported as NaN below
    typename C::XRows xr;
    xr.off[0] = (int64_t)xr_row * a.K;

    f32x4 acc[TT][1];
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[t][0] = zero4();
    if (!bad_e) {
      const int per = (a.chunks + waves - 1) / waves;
      const int c0 = min(wave * per, a.chunks), c1 = min(c0 + per, a.chunks);
      if (c1 > c0) C::run(a.x, xr, r, a.K, c0, c1, acc);
    }

    // sum the wavefronts' partial tiles; element e of tile t < NT (and its up
    // partner at t + NT) -> output (pair p + g0 + m, column n)
    float* mine = lds + wave * C::RED_FLOATS_PER_WAVE;
#pragma unroll
    for (int t = 0; t < TT; ++t)
#pragma unroll
      for (int j = 0; j < 4; ++j) mine[(t * 4 + j) * 64 + lane] = acc[t][0][j];
    __syncthreads();
    constexpr int OUT = NT * 4 * 64;
    for (int el = tid; el < OUT; el += waves * 64) {
      float v = 0.f, u = 0.f;
      for (int w = 0; w < waves; ++w) {
        v += lds[w * C::RED_FLOATS_PER_WAVE + el];
        if (GLU) u += lds[w * C::RED_FLOATS_PER_WAVE + OUT + el];
      }
      const int l = el & 63, j = (el >> 6) & 3, t = el >> 8;
      const int m = 4 * (l >> 4) + j;
      const int n = n0 + t * 16 + (l & 15);
      if (m < rows && n < a.N) {
        const int pp = p + g0 + m;
        const int xrow = a.lhs ? a.lhs[pp] : pp;
        float out;
        if (bad_e || xrow < 0 || xrow >= a.x_rows) {
          out = __builtin_nanf("");
        } else if (GLU) {
          out = silu_mul<Tag>(rnd<Tag>(v), rnd<Tag>(u));
        } else {
          out = v;
        }
        a.y[(int64_t)pp * a.N + n] = Num<Tag>::f2h(out);
      }
    }
    __syncthreads();  // the next group reuses the reduction buffer
  }
}

template <typename Tag, int GS, bool GLU, int SBPC>
__global__ __launch_bounds__(256) void gather_stream_kernel(GatherArgs a) {
  using S = Stream<Tag, GS, 1, 4, SBPC>;
  constexpr int OUTC = GLU ? S::NB / 2 : S::NB;  // output columns per workgroup
  __shared__ int32_t s_rows[16];   // activation row of each MFMA row (clamped)
  __shared__ int32_t s_lhs[16];    // raw lhs ids of the current 16 pairs
  __shared__ int32_t s_rhs[18];    // rhs[p-1 .. p+16]
  const int p = blockIdx.y;
  const int tid = threadIdx.x;
  // One memory round trip for all the indexing: the expert ids around p and
  // the activation rows of the first 16 pairs, loaded together.
  if (tid < 18) {
    const int q = p - 1 + tid;
    s_rhs[tid] = (q >= 0 && q < a.P) ? a.rhs[q] : 0;
  } else if (tid >= 64 && tid < 80) {
    const int q = min(p + tid - 64, a.P - 1);
    s_lhs[tid - 64] = a.lhs ? a.lhs[q] : q;
  }
  __syncthreads();
  const int e = s_rhs[1];
  if (p > 0 && s_rhs[0] == e) return;  // not the first pair of its run (uniform)
  int run = 1;
  while (p + run < a.P && run < 17 && s_rhs[1 + run] == e) ++run;
  if (run == 17)  // a run longer than the window: rare, continue in memory
    while (p + run < a.P && a.rhs[p + run] == e) ++run;
  const bool bad_e = e < 0 || e >= a.E;
  const size_t ee = bad_e ? 0 : (size_t)e;
  const uint32_t wbytes = (uint32_t)a.N * (uint32_t)(a.K / 2);
  const uint32_t sbytes = (uint32_t)a.N * (uint32_t)(a.K / GS) * 2u;
  typename S::Ctx cx;
  cx.x = buffer_rsrc(a.x, (uint32_t)a.x_rows * (uint32_t)a.K * 2u);
  cx.w = buffer_rsrc(a.w[0] + ee * (wbytes / 4), wbytes);
  cx.s = buffer_rsrc(a.s[0] + ee * (sbytes / 2), sbytes);
  cx.b = buffer_rsrc(a.b[0] + ee * (sbytes / 2), sbytes);
  cx.w2 = buffer_rsrc(a.w[1] + ee * (wbytes / 4), wbytes);
  cx.s2 = buffer_rsrc(a.s[1] + ee * (sbytes / 2), sbytes);
  cx.b2 = buffer_rsrc(a.b[1] + ee * (sbytes / 2), sbytes);
  cx.split = GLU ? OUTC : S::NB;
  cx.xrows = s_rows;
  cx.xbase = 0;
  cx.K = a.K;
  cx.N = a.N;
  cx.groups = a.K / GS;
  cx.n0 = blockIdx.x * OUTC;
  cx.lane = tid & 63;
  cx.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  float* red = reinterpret_cast<float*>(dfmi_smem);
  for (int g0 = 0; g0 < run; g0 += 16) {
    const int rows = min(16, run - g0);
    if (g0 > 0 && tid < 16) {  // later row blocks of a long run
      const int pp = p + g0 + min(tid, rows - 1);
      s_lhs[tid] = a.lhs ? a.lhs[pp] : pp;
    }
    __syncthreads();
    if (tid < 16) {
      // rows past the run repeat its last pair; invalid ids read row 0 and
      // are reported as NaN below
      int xr = s_lhs[min(tid, rows - 1)];
      if (xr < 0 || xr >= a.x_rows) xr = 0;
      s_rows[tid] = xr;
    }
    __syncthreads();
    cx.M = rows;
    f32x4 acc[S::NT][1];
#pragma unroll
    for (int t = 0; t < S::NT; ++t) acc[t][0] = zero4();
    if (!bad_e) S::run(cx, 0, a.K / S::CK, acc);
    // sum the 4 wavefronts' partial tiles through LDS (every DMA has landed)
    __syncthreads();
    {
      float* mine = red + cx.wave * S::RED_FLOATS;
#pragma unroll
      for (int t = 0; t < S::NT; ++t)
#pragma unroll
        for (int j = 0; j < 4; ++j) mine[(t * 4 + j) * 64 + cx.lane] = acc[t][0][j];
    }
    __syncthreads();
    constexpr int OUT = OUTC * 16;  // output elements: tiles 0 .. OUTC/16-1
    for (int el = tid; el < OUT; el += 256) {
      float v = 0.f, u = 0.f;
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        v += red[w * S::RED_FLOATS + el];
        if (GLU) u += red[w * S::RED_FLOATS + OUT + el];  // up tile t + OUTC/16
      }
      const int l = el & 63, j = (el >> 6) & 3, t = el >> 8;
      const int m = 4 * (l >> 4) + j;
      const int n = cx.n0 + t * 16 + (l & 15);
      if (m < rows && n < a.N) {
        const int pp = p + g0 + m;
        const int xrow = s_lhs[m];
        float out;
        if (bad_e || xrow < 0 || xrow >= a.x_rows) {
          out = __builtin_nanf("");
        } else if (GLU) {
          out = silu_mul<Tag>(rnd<Tag>(v), rnd<Tag>(u));
        } else {
          out = v;
        }
        a.y[(int64_t)pp * a.N + n] = Num<Tag>::f2h(out);
      }
    }
    __syncthreads();  // s_lhs, s_rows and the LDS stages are reused by the next row block
  }
}

template <typename Tag, int GS, bool GLU, int SBPC>
static void launch_gather_stream_t(const GatherArgs& a, hipStream_t st) {
  using S = Stream<Tag, GS, 1, 4, SBPC>;
  constexpr int OUTC = GLU ? S::NB / 2 : S::NB;
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&gather_stream_kernel<Tag, GS, GLU, SBPC>),
      hipFuncAttributeMaxDynamicSharedMemorySize, S::LDS_BYTES);
  (void)attr;
  const dim3 grid((unsigned)((a.N + OUTC - 1) / OUTC), (unsigned)a.P);
  hipLaunchKernelGGL((gather_stream_kernel<Tag, GS, GLU, SBPC>), grid, dim3(256), S::LDS_BYTES,
                     st, a);
}

// The narrow scale window (8 pieces, 64 KB of LDS with 4 wavefronts) keeps
// two workgroups per CU next to the kernel's static index arrays; K ranges
// of more groups take the wide one (80 KB, one workgroup per CU).
template <typename Tag, bool GLU, int GS>
static void launch_gather_stream_gs(const GatherArgs& a, hipStream_t st) {
  if (a.K / GS <= sb_max_groups(8)) launch_gather_stream_t<Tag, GS, GLU, 8>(a, st);
  else launch_gather_stream_t<Tag, GS, GLU, kSbPieces>(a, st);
}

template <typename Tag, bool GLU>
static void launch_gather_stream(const GatherArgs& a, int gs, hipStream_t st) {
  if (gs == 32) launch_gather_stream_gs<Tag, GLU, 32>(a, st);
  else if (gs == 64) launch_gather_stream_gs<Tag, GLU, 64>(a, st);
  else launch_gather_stream_gs<Tag, GLU, 128>(a, st);
}

template <typename Tag, int GS, int NT, bool KFULL, bool GLU>
static void launch_gather_t(const GatherArgs& a, int n_blocks, int waves, hipStream_t st) {
  hipLaunchKernelGGL((gather_kernel<Tag, GS, NT, KFULL, GLU>), dim3(n_blocks, a.P),
                     dim3(64 * waves), 0, st, a);
}

template <typename Tag, int GS, bool GLU>
static void launch_gather_gs(const GatherArgs& a, bool kfull, int nt, int n_blocks, int waves,
                             hipStream_t st) {
  if (nt == 1) {
    if (kfull) launch_gather_t<Tag, GS, 1, true, GLU>(a, n_blocks, waves, st);
    else launch_gather_t<Tag, GS, 1, false, GLU>(a, n_blocks, waves, st);
  } else {
    if (kfull) launch_gather_t<Tag, GS, 2, true, GLU>(a, n_blocks, waves, st);
    else launch_gather_t<Tag, GS, 2, false, GLU>(a, n_blocks, waves, st);
  }
}

template <typename Tag, bool GLU>
static void launch_gather(const GatherArgs& a, int gs, bool kfull, int nt, int n_blocks,
                          int waves, hipStream_t st) {
  if (gs == 32) launch_gather_gs<Tag, 32, GLU>(a, kfull, nt, n_blocks, waves, st);
  else if (gs == 64) launch_gather_gs<Tag, 64, GLU>(a, kfull, nt, n_blocks, waves, st);
  else launch_gather_gs<Tag, 128, GLU>(a, kfull, nt, n_blocks, waves, st);
}

static int validate_gather(int x_dtype, int64_t x_rows, int64_t P, int64_t K, int64_t N,
                           int64_t E, int gs, int bits) {
  if (x_dtype != DFMI_BF16 && x_dtype != DFMI_F16) {
    set_error("dfmi_gather_qmm: x dtype %d unsupported (bf16 or f16)", x_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4) {
    set_error("dfmi_gather_qmm: bits=%d unsupported (4)", bits);
    return DFMI_EINVAL;
  }
  if (gs != 32 && gs != 64 && gs != 128) {
    set_error("dfmi_gather_qmm: group_size=%d unsupported (32, 64, 128)", gs);
    return DFMI_EINVAL;
  }
  if (P < 0 || N < 0 || E < 1 || x_rows < 1 || K < 32 || K % 32 || K % gs) {
    set_error("dfmi_gather_qmm: bad shape P=%lld K=%lld N=%lld E=%lld x_rows=%lld gs=%d",
              (long long)P, (long long)K, (long long)N, (long long)E, (long long)x_rows, gs);
    return DFMI_EINVAL;
  }
  if (P > 65535 || N >= (1ll << 31) || K >= (1ll << 31) || x_rows >= (1ll << 31) ||
      N * (K / 8) > 0xFFFFFFFFll) {
    set_error("dfmi_gather_qmm: shape too large P=%lld K=%lld N=%lld", (long long)P,
              (long long)K, (long long)N);
    return DFMI_EINVAL;
  }
  return DFMI_OK;
}

static int gather_common(const void* x, int x_dtype, int64_t x_rows, const uint32_t* w0,
                         const void* s0, const void* b0, const uint32_t* w1, const void* s1,
                         const void* b1, const int32_t* lhs_rows, const int32_t* rhs_experts,
                         void* y, int64_t P, int64_t K, int64_t N, int64_t E, int group_size,
                         int bits, bool glu, void* stream) {
  int rc = validate_gather(x_dtype, x_rows, P, K, N, E, group_size, bits);
  if (rc != DFMI_OK) return rc;
  if (P == 0 || N == 0) return DFMI_OK;
  if (!x || !w0 || !s0 || !b0 || !rhs_experts || !y || (glu && (!w1 || !s1 || !b1))) {
    set_error("dfmi_gather_qmm: null pointer");
    return DFMI_EINVAL;
  }
  if (!aligned16(x) || !aligned16(w0) || !aligned16(s0) || !aligned16(b0) ||
      (glu && (!aligned16(w1) || !aligned16(s1) || !aligned16(b1)))) {
    set_error("dfmi_gather_qmm: x, weights, scales and biases must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  GatherArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.x_rows = x_rows;
  a.w[0] = w0;
  a.s[0] = static_cast<const uint16_t*>(s0);
  a.b[0] = static_cast<const uint16_t*>(b0);
  a.w[1] = glu ? w1 : w0;
  a.s[1] = static_cast<const uint16_t*>(glu ? s1 : s0);
  a.b[1] = static_cast<const uint16_t*>(glu ? b1 : b0);
  a.lhs = lhs_rows;
  a.rhs = rhs_experts;
  a.y = static_cast<uint16_t*>(y);
  a.P = (int)P;
  a.K = (int)K;
  a.N = (int)N;
  a.E = (int)E;
  a.chunks = (int)((K + kChunkK - 1) / kChunkK);
  hipStream_t st = static_cast<hipStream_t>(stream);
  // streaming loop: whole 256-k steps, the whole K in one scale / bias
  // window, 32-bit buffer offsets per expert and for the activations.
  // Measured on MI355X (16 tokens, top-8 of 256 experts): equal to the
  // general loop for the SwiGLU pair at K = 2048 and slower for K = 512 (two
  // steps per workgroup do not amortise its pipeline fill), so short K stays
  // on the general loop.
  if (stream_eligible(16, K, N, group_size) && K >= 1024 && x_rows * K * 2 < (1ll << 31) &&
      K / group_size <= sb_max_groups(kSbPieces)) {
    if (glu) {
      if (x_dtype == DFMI_BF16) launch_gather_stream<BF16, true>(a, group_size, st);
      else launch_gather_stream<F16, true>(a, group_size, st);
    } else {
      if (x_dtype == DFMI_BF16) launch_gather_stream<BF16, false>(a, group_size, st);
      else launch_gather_stream<F16, false>(a, group_size, st);
    }
    return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
  }
  const bool kfull = (K % kChunkK) == 0;
  const int nt = N >= 1024 ? 2 : 1;
  const int n_blocks = (int)((N + 16 * nt - 1) / (16 * nt));
  const int waves = std::max(1, std::min(kMaxWaves, a.chunks));
  if (glu) {
    if (x_dtype == DFMI_BF16) launch_gather<BF16, true>(a, group_size, kfull, nt, n_blocks, waves, st);
    else launch_gather<F16, true>(a, group_size, kfull, nt, n_blocks, waves, st);
  } else {
    if (x_dtype == DFMI_BF16) launch_gather<BF16, false>(a, group_size, kfull, nt, n_blocks, waves, st);
    else launch_gather<F16, false>(a, group_size, kfull, nt, n_blocks, waves, st);
  }
  return check_launch(glu ? "dfmi_gather_qmm_swiglu" : "dfmi_gather_qmm_affine");
}

// out[t, d] = rnd(sum_j scores[t, j] * y[r(t*k + j), d]), fp32, j in order;
// r(p) = y_rows[p] (the pair's row in a sorted y: the unsort mlx-lm's
// SwitchGLU applies before the weighted sum) or p.  A row id outside
// [0, T*k) makes the output NaN.
template <typename Tag>
__global__ __launch_bounds__(256) void combine_kernel(const uint16_t* y, const int32_t* y_rows,
                                                      const float* scores, uint16_t* out, int T,
                                                      int k, int D) {
  const int t = blockIdx.y;
  const int64_t P = (int64_t)T * k;
  for (int d = blockIdx.x * 256 + threadIdx.x; d < D; d += gridDim.x * 256) {
    float acc = 0.f;
    for (int j = 0; j < k; ++j) {
      const int64_t p = (int64_t)t * k + j;
      const int64_t r = y_rows ? (int64_t)y_rows[p] : p;
      const float v = (r >= 0 && r < P) ? Num<Tag>::h2f(y[r * D + d]) : __builtin_nanf("");
      acc = __builtin_fmaf(scores[p], v, acc);
    }
    out[(int64_t)t * D + d] = Num<Tag>::f2h(acc);
  }
}

}  // namespace dfmi

using namespace dfmi;

extern "C" int dfmi_gather_qmm_affine(const void* x, int x_dtype, int64_t x_rows,
                                      const uint32_t* w_q, const void* scales, const void* biases,
                                      const int32_t* lhs_rows, const int32_t* rhs_experts,
                                      void* y, int64_t P, int64_t K, int64_t N, int64_t E,
                                      int group_size, int bits, void* stream) {
  return gather_common(x, x_dtype, x_rows, w_q, scales, biases, nullptr, nullptr, nullptr,
                       lhs_rows, rhs_experts, y, P, K, N, E, group_size, bits, false, stream);
}

extern "C" int dfmi_gather_qmm_swiglu(const void* x, int x_dtype, int64_t x_rows,
                                      const uint32_t* wg_q, const void* g_scales,
                                      const void* g_biases, const uint32_t* wu_q,
                                      const void* u_scales, const void* u_biases,
                                      const int32_t* lhs_rows, const int32_t* rhs_experts,
                                      void* h, int64_t P, int64_t K, int64_t N, int64_t E,
                                      int group_size, int bits, void* stream) {
  return gather_common(x, x_dtype, x_rows, wg_q, g_scales, g_biases, wu_q, u_scales, u_biases,
                       lhs_rows, rhs_experts, h, P, K, N, E, group_size, bits, true, stream);
}

extern "C" int dfmi_moe_combine(const void* y, int y_dtype, const int32_t* y_rows,
                                const float* scores, void* out, int64_t T, int64_t k, int64_t D,
                                void* stream) {
  if (y_dtype != DFMI_BF16 && y_dtype != DFMI_F16) {
    set_error("dfmi_moe_combine: dtype %d unsupported (bf16 or f16)", y_dtype);
    return DFMI_EINVAL;
  }
  if (T < 0 || k < 1 || D < 0 || T > 65535 || T * k * D >= (1ll << 40)) {
    set_error("dfmi_moe_combine: bad shape T=%lld k=%lld D=%lld", (long long)T, (long long)k,
              (long long)D);
    return DFMI_EINVAL;
  }
  if (T == 0 || D == 0) return DFMI_OK;
  if (!y || !scores || !out) {
    set_error("dfmi_moe_combine: null pointer");
    return DFMI_EINVAL;
  }
  const int gx = (int)std::min<int64_t>((D + 255) / 256, 64);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (y_dtype == DFMI_BF16)
    hipLaunchKernelGGL(combine_kernel<BF16>, dim3(gx, (unsigned)T), dim3(256), 0, st,
                       static_cast<const uint16_t*>(y), y_rows, scores,
                       static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
  else
    hipLaunchKernelGGL(combine_kernel<F16>, dim3(gx, (unsigned)T), dim3(256), 0, st,
                       static_cast<const uint16_t*>(y), y_rows, scores,
                       static_cast<uint16_t*>(out), (int)T, (int)k, (int)D);
  return check_launch("dfmi_moe_combine");
}
