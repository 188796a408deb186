// Dense affine int4 qmm: y[M,N] = x[M,K] . dequant(W)^T on gfx950.
//
// Grid: one workgroup (4 wavefronts) per (output block of 64*NT columns,
// K split).  Each wavefront owns NT 16-column tiles of the block and all M
// rows (MT 16-row MFMA blocks, M <= 32; larger M tiles over grid.y).  When a
// block is split along K over `kpg` workgroups, each writes an fp32 partial
// and the last one to finish (atomic counter) sums the partials in split
// order -- the result does not depend on arrival order -- and writes y.  The
// splits of one block are mapped to one XCD (workgroup ids are dealt to the 8
// XCDs round-robin) so the partials stay in that XCD's L2.
#include <algorithm>
#include <cmath>

#include "dfmi_core.h"
#include "dfmi_host.h"

namespace dfmi {

struct DenseArgs {
  const uint16_t* x;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  uint16_t* y;
  float* partials;
  uint32_t* counters;
  int M, K, N;
  int kpg;       // workgroups sharing one output block along K
  int chunks;    // ceil(K / 256)
  int n_blocks;  // ceil(N / (64 * NT))
  int xcd_map;   // 1: the K splits of a block are dealt to the same XCD
};

template <typename Tag, int GS, int MT, int NT, bool KFULL>
__global__ __launch_bounds__(kThreads) void qmm_dense_kernel(DenseArgs a) {
  using C = Core<Tag, GS, MT, NT, KFULL>;
  constexpr int NB = kWaves * 16 * NT;
  __shared__ __attribute__((aligned(16))) char lds[C::LDS_BYTES];
  __shared__ int s_last;

  int nb, kp;
  {
    const int L = blockIdx.x;
    if (a.xcd_map) {
      const int xcd = L & 7, j = L >> 3;
      const int nbl = j / a.kpg;
      kp = j - nbl * a.kpg;
      nb = nbl * 8 + xcd;
    } else {
      nb = L / a.kpg;
      kp = L - nb * a.kpg;
    }
  }
  if (nb >= a.n_blocks) return;  // uniform for the block, before any barrier

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int m_base = blockIdx.y * 16 * MT;
  const uint32_t kw = (uint32_t)(a.K / 8);
  const uint32_t kgrp = (uint32_t)(a.K / GS);

  typename C::Stage st;
#pragma unroll
  for (int i = 0; i < C::SPT; ++i) {
    const int slot = tid + kThreads * i;
    int m, kk;
    C::slot_geometry(slot, m, kk);
    const int mm = m_base + m;
    st.xoff[i] = mm < a.M ? (int64_t)mm * a.K : -1;
    st.kk[i] = kk;
    st.lds[i] = slot * 16;
  }

  const int col0 = nb * NB + wave * 16 * NT;
  typename C::Rows r;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = min(col0 + t * 16 + (lane & 15), a.N - 1);
    r.wbase[t] = a.w;
    r.sbase[t] = a.s;
    r.bbase[t] = a.b;
    r.woff[t] = (uint32_t)row * kw;
    r.soff[t] = (uint32_t)row * kgrp;
  }

  const int c_begin = (int)((int64_t)kp * a.chunks / a.kpg);
  const int c_end = (int)((int64_t)(kp + 1) * a.chunks / a.kpg);
  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4();

  C::run(a.x, st, r, a.K, c_begin, c_end, lds, acc);

  const int kg = lane >> 4, col = lane & 15;
  if (a.kpg == 1) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      const int n = col0 + t * 16 + col;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int m = m_base + mt * 16 + 4 * kg + j;
          if (m < a.M && n < a.N) a.y[(int64_t)m * a.N + n] = Num<Tag>::f2h(acc[t][mt][j]);
        }
    }
    return;
  }

  // K split: publish this split's partial, the last arriver reduces.
  float* part = a.partials + (int64_t)kp * a.M * a.N;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int n = col0 + t * 16 + col;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = mt * 16 + 4 * kg + j;  // M <= 32 on this path (grid.y == 1)
        if (m < a.M && n < a.N) part[(int64_t)m * a.N + n] = acc[t][mt][j];
      }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&a.counters[nb], 1u);
    s_last = (prev == (unsigned)(a.kpg - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  const int n0 = nb * NB;
  for (int idx = tid; idx < a.M * NB; idx += kThreads) {
    const int m = idx / NB, n = n0 + idx % NB;
    if (n < a.N) {
      float sum = 0.f;
      for (int q = 0; q < a.kpg; ++q) sum += a.partials[((int64_t)q * a.M + m) * a.N + n];
      a.y[(int64_t)m * a.N + n] = Num<Tag>::f2h(sum);
    }
  }
  if (tid == 0) a.counters[nb] = 0u;
}

// Counters live in a fixed-size region at the start of every qmm workspace,
// so calls of different shapes agree on where they are (a counter is only
// ever zero between calls).
constexpr size_t kCounterBytes = 65536;
constexpr int kMaxCounters = (int)(kCounterBytes / 4);

struct DensePlan {
  int MT, NT, kpg, chunks, n_blocks, grid_x, grid_y, xcd_map;
  bool kfull;
  size_t counters_bytes, ws_bytes;
};

static int plan_dense(int64_t M, int64_t K, int64_t N, const dfmi_qmm_tuning* tune, DensePlan& p) {
  p.MT = M <= 16 ? 1 : 2;
  p.grid_y = M <= 32 ? 1 : (int)((M + 31) / 32);
  p.chunks = (int)((K + kChunkK - 1) / kChunkK);
  p.kfull = (K % kChunkK) == 0;
  int nt = (tune && tune->tiles_per_wave) ? tune->tiles_per_wave : (((N + 127) / 128) >= 64 ? 2 : 1);
  if (nt != 1 && nt != 2) {
    set_error("dfmi_qmm: tiles_per_wave must be 1 or 2 (got %d)", nt);
    return DFMI_EINVAL;
  }
  p.NT = nt;
  const int64_t nb_cols = (int64_t)kWaves * 16 * nt;
  p.n_blocks = (int)((N + nb_cols - 1) / nb_cols);
  int kpg;
  if (M > 32) {
    kpg = 1;
  } else if (tune && tune->k_splits > 0) {
    kpg = tune->k_splits;
  } else {
    kpg = (int)std::lround(512.0 / (double)p.n_blocks);
    kpg = std::min(kpg, std::max(1, p.chunks / 2));
  }
  p.kpg = std::max(1, std::min(kpg, p.chunks));
  if (p.n_blocks > kMaxCounters) p.kpg = 1;
  p.xcd_map = (p.n_blocks % 8 == 0) ? 1 : 0;
  p.grid_x = p.n_blocks * p.kpg;
  if (p.kpg > 1) {
    p.counters_bytes = kCounterBytes;
    p.ws_bytes = p.counters_bytes + (size_t)p.kpg * (size_t)M * (size_t)N * 4u;
  } else {
    p.counters_bytes = 0;
    p.ws_bytes = 0;
  }
  return DFMI_OK;
}

template <typename Tag, int GS, int MT, int NT>
static void launch_kf(bool kfull, dim3 g, hipStream_t st, const DenseArgs& a) {
  if (kfull)
    hipLaunchKernelGGL((qmm_dense_kernel<Tag, GS, MT, NT, true>), g, dim3(kThreads), 0, st, a);
  else
    hipLaunchKernelGGL((qmm_dense_kernel<Tag, GS, MT, NT, false>), g, dim3(kThreads), 0, st, a);
}

template <typename Tag, int GS>
static void launch_gs(const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  const dim3 g(p.grid_x, p.grid_y);
  if (p.MT == 1) {
    if (p.NT == 1) launch_kf<Tag, GS, 1, 1>(p.kfull, g, st, a);
    else launch_kf<Tag, GS, 1, 2>(p.kfull, g, st, a);
  } else {
    if (p.NT == 1) launch_kf<Tag, GS, 2, 1>(p.kfull, g, st, a);
    else launch_kf<Tag, GS, 2, 2>(p.kfull, g, st, a);
  }
}

template <typename Tag>
static void launch_tag(int gs, const DensePlan& p, hipStream_t st, const DenseArgs& a) {
  if (gs == 32) launch_gs<Tag, 32>(p, st, a);
  else if (gs == 64) launch_gs<Tag, 64>(p, st, a);
  else launch_gs<Tag, 128>(p, st, a);
}

static int validate_qmm(int x_dtype, int64_t M, int64_t K, int64_t N, int gs, int bits) {
  if (x_dtype != DFMI_BF16 && x_dtype != DFMI_F16) {
    set_error("dfmi_qmm: x dtype %d unsupported (bf16 or f16)", x_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4) {
    set_error("dfmi_qmm: bits=%d unsupported (4)", bits);
    return DFMI_EINVAL;
  }
  if (gs != 32 && gs != 64 && gs != 128) {
    set_error("dfmi_qmm: group_size=%d unsupported (32, 64, 128)", gs);
    return DFMI_EINVAL;
  }
  if (M < 0 || N < 0 || K < 32 || K % 32 || K % gs) {
    set_error("dfmi_qmm: bad shape M=%lld K=%lld N=%lld gs=%d", (long long)M, (long long)K,
              (long long)N, gs);
    return DFMI_EINVAL;
  }
  if (M >= (1ll << 31) || N >= (1ll << 31) || K >= (1ll << 31) ||
      N * (K / 8) > 0xFFFFFFFFll) {
    set_error("dfmi_qmm: shape too large M=%lld K=%lld N=%lld", (long long)M, (long long)K,
              (long long)N);
    return DFMI_EINVAL;
  }
  return DFMI_OK;
}

}  // namespace dfmi

using namespace dfmi;

extern "C" size_t dfmi_qmm_workspace_bytes_ex(int64_t M, int64_t K, int64_t N, int group_size,
                                              int bits, const dfmi_qmm_tuning* tuning) {
  if (validate_qmm(DFMI_BF16, M, K, N, group_size, bits) != DFMI_OK || M == 0 || N == 0) return 0;
  DensePlan p;
  if (plan_dense(M, K, N, tuning, p) != DFMI_OK) return 0;
  return p.ws_bytes;
}

extern "C" size_t dfmi_qmm_workspace_bytes(int64_t M, int64_t K, int64_t N, int group_size,
                                           int bits) {
  return dfmi_qmm_workspace_bytes_ex(M, K, N, group_size, bits, nullptr);
}

extern "C" int dfmi_qmm_affine_ex(const void* x, int x_dtype, const uint32_t* w_q,
                                  const void* scales, const void* biases, void* y, int64_t M,
                                  int64_t K, int64_t N, int group_size, int bits, void* workspace,
                                  size_t workspace_bytes, const dfmi_qmm_tuning* tuning,
                                  void* stream) {
  int rc = validate_qmm(x_dtype, M, K, N, group_size, bits);
  if (rc != DFMI_OK) return rc;
  if (M == 0 || N == 0) return DFMI_OK;
  if (!x || !w_q || !scales || !biases || !y) {
    set_error("dfmi_qmm: null pointer");
    return DFMI_EINVAL;
  }
  if (!aligned16(x) || !aligned16(w_q) || !aligned16(scales) || !aligned16(biases)) {
    set_error("dfmi_qmm: x, w_q, scales and biases must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  DensePlan p;
  rc = plan_dense(M, K, N, tuning, p);
  if (rc != DFMI_OK) return rc;
  DenseArgs a;
  a.x = static_cast<const uint16_t*>(x);
  a.w = w_q;
  a.s = static_cast<const uint16_t*>(scales);
  a.b = static_cast<const uint16_t*>(biases);
  a.y = static_cast<uint16_t*>(y);
  a.partials = nullptr;
  a.counters = nullptr;
  if (p.kpg > 1) {
    if (!workspace || workspace_bytes < p.ws_bytes || !aligned16(workspace)) {
      set_error("dfmi_qmm: workspace of %zu bytes (16-byte aligned) required, got %zu",
                p.ws_bytes, workspace_bytes);
      return DFMI_ENOSPC;
    }
    a.counters = static_cast<uint32_t*>(workspace);
    a.partials = reinterpret_cast<float*>(static_cast<char*>(workspace) + p.counters_bytes);
  }
  a.M = (int)M;
  a.K = (int)K;
  a.N = (int)N;
  a.kpg = p.kpg;
  a.chunks = p.chunks;
  a.n_blocks = p.n_blocks;
  a.xcd_map = p.xcd_map;
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (x_dtype == DFMI_BF16) launch_tag<BF16>(group_size, p, st, a);
  else launch_tag<F16>(group_size, p, st, a);
  return check_launch("dfmi_qmm_affine");
}

extern "C" int dfmi_qmm_affine(const void* x, int x_dtype, const uint32_t* w_q, const void* scales,
                               const void* biases, void* y, int64_t M, int64_t K, int64_t N,
                               int group_size, int bits, void* workspace, size_t workspace_bytes,
                               void* stream) {
  return dfmi_qmm_affine_ex(x, x_dtype, w_q, scales, biases, y, M, K, N, group_size, bits,
                            workspace, workspace_bytes, nullptr, stream);
}
