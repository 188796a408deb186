// Greedy verify on gfx950: argmax over the vocabulary per verify row, accept
// length against the drafted block, bonus token.
//
//  * lmhead_stream_kernel: the lm_head matmul on the streaming main loop (64
//    vocabulary rows per workgroup, the whole K, LDS-DMA staging) whose
//    epilogue rounds each logit to the activation dtype (the dtype the
//    reference's logits carry), applies the optional Gemma softcap and the
//    suppress mask, and reduces to a per-row (value, index) argmax key.  The
//    logits never reach HBM unless the caller asks for them.
//  * lmhead_greedy_kernel: the same on the general main loop, for shapes the
//    streaming loop does not take (K not a multiple of 256 or of 8 groups).
//  * greedy_kernel: the same reduction over logits already in memory.
//
// Cross-workgroup reduction: a 64-bit key (monotone value bits << 32 |
// ~index) per row, combined with a device-scope atomic max -- max is
// order-independent, so the winner (largest value, then lowest index) is
// deterministic.  All cross-workgroup communication is atomic
// read-modify-writes on the workspace: every workgroup waits for its key
// RMWs to return before its counter RMW, and the workgroup whose counter RMW
// returns total-1 (the last) reads each key with an exchange that also
// clears it, computes accept / bonus and clears the counter.  No plain
// store is published across workgroups, so no cache writeback or invalidate
// (the cost of a device-scope fence on this GPU) is needed.
#include <math.h>

#include "dfmi_core.h"
#include "dfmi_host.h"
#include "dfmi_stream.h"

namespace dfmi {

constexpr int kMaxGreedyRows = 32;
constexpr int kGreedyThreads = 256;

struct GreedyOut {
  unsigned long long* keys;  // [M] workspace, zero between calls
  uint32_t* counter;         // workspace, zero between calls
  uint32_t* posterior;       // [M]
  int32_t* accept_len;       // [1] or null
  uint32_t* bonus;           // [1] or null
  const uint32_t* verify_ids;  // [M] or null
  int M;
};

__device__ inline unsigned long long umax64(unsigned long long a, unsigned long long b) {
  return a > b ? a : b;
}

// LDS scratch of greedy_publish_and_finish (the caller places it: a static
// __shared__ object, or a slice of a kernel's dynamic LDS).
struct GreedyLds {
  int last;
  int sink;
  uint32_t post[kMaxGreedyRows];
};

// Publish this workgroup's keys for rows [r0, r1) (s_best[m] in LDS) and, in
// the last workgroup to arrive, turn the keys into tokens, accept and bonus.
__device__ inline void greedy_publish_and_finish(const GreedyOut& o,
                                                 const unsigned long long* s_best, int r0,
                                                 int r1, unsigned total_blocks, GreedyLds* g) {
  int& s_last = g->last;
  int& s_sink = g->sink;
  uint32_t* s_post = g->post;
  const int tid = threadIdx.x;
  if (tid >= r0 && tid < r1) {
    const unsigned long long old = __hip_atomic_fetch_max(
        &o.keys[tid], s_best[tid], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (old == ~0ull) s_sink = 1;  // consume the result: the RMW has completed
  }
  __syncthreads();
  if (tid == 0) {
    const unsigned prev =
        __hip_atomic_fetch_add(o.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = (prev == total_blocks - 1) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  if (tid < o.M) {
    const unsigned long long k =
        __hip_atomic_exchange(&o.keys[tid], 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const uint32_t tok = key_index(k);
    s_post[tid] = tok;
    o.posterior[tid] = tok;
  }
  __syncthreads();
  if (tid == 0) {
    if (o.verify_ids != nullptr) {
      int a = 0;
      while (a + 1 < o.M && o.verify_ids[a + 1] == s_post[a]) ++a;
      if (o.accept_len) o.accept_len[0] = a;
      if (o.bonus) o.bonus[0] = s_post[a];
    }
    __hip_atomic_exchange(o.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <typename Tag>
__device__ inline float round_t(float v) {
  return Num<Tag>::h2f(Num<Tag>::f2h(v));
}

// logit value as the reference sees it: rounded to the dtype, optionally
// softcapped with op-by-op rounding (target_gemma4.py:33-40).
template <typename Tag>
__device__ inline float logit_value(float acc, float capr) {
  float v = round_t<Tag>(acc);
  if (capr > 0.f) {
    const float t1 = round_t<Tag>(v / capr);
    const float t2 = round_t<Tag>(tanhf(t1));
    v = round_t<Tag>(t2 * capr);
  }
  return v;
}

struct LmArgs {
  const uint16_t* h;
  const uint32_t* w;
  const uint16_t* s;
  const uint16_t* b;
  const uint32_t* t;  // [K/gs][V] (scale, bias) pairs (pair-streaming kernel) or null
  const uint8_t* mask;
  uint16_t* logits;  // [M, V] or null
  float softcap;
  int M, K, V;
  int chunks;
  int n_blocks;
  GreedyOut out;
};

constexpr int kLmTiles = 4;  // 64 vocabulary rows per workgroup
static_assert(16 * kLmTiles == kStreamRows, "one block numbering for both lm_head kernels");

template <typename Tag, int GS, int MT, bool KFULL>
__global__ __launch_bounds__(kMaxWaves * 64) void lmhead_greedy_kernel(LmArgs a) {
  constexpr int NT = kLmTiles;
  using C = Core<Tag, GS, MT, NT, KFULL>;
  __shared__ __attribute__((aligned(16))) float lds[C::LDS_BYTES / 4];
  __shared__ unsigned long long s_best[16 * MT];

  const int tid = threadIdx.x, lane = tid & 63;
  // wave-uniform values in scalar registers, so the chunk loop is a scalar loop
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int waves = blockDim.x >> 6;
  const int n0 = blockIdx.x * 16 * NT;
  if (tid < 16 * MT) s_best[tid] = 0ull;

  const typename C::XRows xr = C::x_rows(0, a.M, a.K, lane);
  const uint32_t kw = (uint32_t)(a.K / 8);
  const uint32_t kgrp = (uint32_t)(a.K / GS);
  typename C::Rows r;
#pragma unroll
  for (int t = 0; t < NT; ++t) {
    const int row = min(n0 + t * 16 + (lane & 15), a.V - 1);
    r.wbase[t] = a.w;
    r.sbase[t] = a.s;
    r.bbase[t] = a.b;
    r.woff[t] = (uint32_t)row * kw;
    r.soff[t] = (uint32_t)row * kgrp;
  }
  f32x4 acc[NT][MT];
#pragma unroll
  for (int t = 0; t < NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4();
  const int kr = (wave + (int)blockIdx.x) % waves;
  const int c0 = kr * a.chunks / waves;
  const int c1 = (kr + 1) * a.chunks / waves;
  if (c1 > c0) C::run(a.h, xr, r, a.K, c0, c1, acc);

  const float capr = a.softcap > 0.f ? round_t<Tag>(a.softcap) : 0.f;
  const float neg = round_t<Tag>(-1e9f);
  C::reduce(lds, acc, waves, [&](int t, int mt, int j, int l, float sum) {
    const int m = mt * 16 + 4 * (l >> 4) + j;
    const int n = n0 + t * 16 + (l & 15);
    if (m < a.M && n < a.V) {
      float v = logit_value<Tag>(sum, capr);
      if (a.logits) a.logits[(int64_t)m * a.V + n] = Num<Tag>::f2h(v);
      if (a.mask && a.mask[n]) v = neg;
      atomicMax(&s_best[m], argmax_key(v, (uint32_t)n));
    }
  });
  __syncthreads();
  __shared__ GreedyLds s_g;
  greedy_publish_and_finish(a.out, s_best, 0, a.M, (unsigned)a.n_blocks, &s_g);
}

// TSB / RW: the pair-streaming main loop with 128-row blocks (two row groups
// of 4 wavefronts sharing the activation stage); the window loop otherwise.
template <typename Tag, int GS, int MT, int WV, bool TSB = false, int RW = 1>
__global__ __launch_bounds__(64 * WV) void lmhead_stream_kernel(
    const uint16_t* h, const uint32_t* w, const uint32_t* t, const uint16_t* s,
    const uint16_t* b, int M, int K, int V, const uint8_t* mask, uint16_t* logits,
    float softcap, int chunks, int n_blocks, unsigned long long* keys, uint32_t* counter,
    uint32_t* posterior, int32_t* accept_len, uint32_t* bonus, const uint32_t* verify_ids,
    int out_M) {
  // Scalar arguments, what the first DMA needs first: the hardware preloads
  // the first 14 dwords into SGPRs (h, w, t, s, b, M, K, V), so a workgroup
  // starts its loads without a scalar-load round trip; the rest is first
  // needed by the epilogue.
  const LmArgs a{h,    w,     s,    b,   t,        mask,     logits,
                 softcap, M, K, V, chunks, n_blocks,
                 GreedyOut{keys, counter, posterior, accept_len, bonus, verify_ids, out_M}};
  using S = Stream<Tag, GS, MT, WV, kSbPieces, 4, RW, TSB>;
  constexpr int kThreads = 64 * WV;
  // Dynamic LDS only (two workgroups of 4 wavefronts fill a CU's LDS): the
  // epilogue's argmax keys and greedy scratch follow the reduction buffer.
  static_assert(WV * S::RED_FLOATS * 4 + 16 * MT * 8 + sizeof(GreedyLds) <= S::LDS_BYTES,
                "epilogue LDS");
  unsigned long long* s_best =
      reinterpret_cast<unsigned long long*>(dfmi_smem + WV * S::RED_FLOATS * 4);
  GreedyLds* s_g = reinterpret_cast<GreedyLds*>(s_best + 16 * MT);
  const int tid = threadIdx.x;
  typename S::Ctx cx;
  cx.x = buffer_rsrc(a.h, (uint32_t)a.M * (uint32_t)a.K * 2u);
  cx.w = buffer_rsrc(a.w, (uint32_t)a.V * (uint32_t)(a.K / 2));
  cx.s = buffer_rsrc(a.s, (uint32_t)a.V * (uint32_t)(a.K / GS) * 2u);
  cx.b = buffer_rsrc(a.b, (uint32_t)a.V * (uint32_t)(a.K / GS) * 2u);
  if constexpr (TSB) cx.t = buffer_rsrc(a.t, (uint32_t)a.V * (uint32_t)(a.K / GS) * 4u);
  cx.K = a.K;
  cx.M = a.M;
  cx.N = a.V;
  cx.groups = a.K / GS;
  cx.n0 = blockIdx.x * S::NB;
  cx.lane = tid & 63;
  cx.wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  cx.dense();
  f32x4 acc[S::NT][MT];
#pragma unroll
  for (int t = 0; t < S::NT; ++t)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[t][mt] = zero4();
  S::template run<true>(cx, 0, a.K / S::CK, acc);  // bias terms batched into MFMAs

  // sum the partial tiles of each row group's KW wavefronts through LDS (the
  // stages are free: every DMA has landed and every wavefront is past its
  // last LDS read), in k-slice order
  __syncthreads();
  float* red = reinterpret_cast<float*>(dfmi_smem);
  {
    float* mine = red + cx.wave * S::RED_FLOATS;
#pragma unroll
    for (int t = 0; t < S::NT; ++t)
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int j = 0; j < 4; ++j) mine[((t * MT + mt) * 4 + j) * 64 + cx.lane] = acc[t][mt][j];
  }
  if (tid < 16 * MT) s_best[tid] = 0ull;
  __syncthreads();
  const float capr = a.softcap > 0.f ? round_t<Tag>(a.softcap) : 0.f;
  const float neg = round_t<Tag>(-1e9f);
  // Every element a thread visits has its row m = 16 mt + 4 (lane >> 4) + j
  // with j = wave & 3 (kThreads is a multiple of 256): the thread keeps one
  // best key per activation block, the 16 lanes of a row group combine
  // theirs, and one lane per row updates the workgroup's key in LDS.
  constexpr int PER = RW * S::RED_FLOATS / kThreads;
  unsigned long long best[MT];
#pragma unroll
  for (int u = 0; u < MT; ++u) best[u] = 0ull;
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int e = q * kThreads + tid;
    const int rg = e / S::RED_FLOATS, eo = e % S::RED_FLOATS;
    const float* rr = red + rg * S::KW * S::RED_FLOATS + eo;
    float sum = rr[0];
#pragma unroll
    for (int k = 1; k < S::KW; ++k) sum += rr[k * S::RED_FLOATS];
    const int l = eo & 63, j = (eo >> 6) & 3, tm = eo >> 8;
    const int n = cx.n0 + kStreamRows * rg + (tm / MT) * 16 + (l & 15);
    const int m = (tm % MT) * 16 + 4 * (l >> 4) + j;
    if (m < a.M && n < a.V) {
      float v = logit_value<Tag>(sum, capr);
      if (a.logits) a.logits[(int64_t)m * a.V + n] = Num<Tag>::f2h(v);
      if (a.mask && a.mask[n]) v = neg;
      const unsigned long long key = argmax_key(v, (uint32_t)n);
#pragma unroll
      for (int u = 0; u < MT; ++u)
        if (u == tm % MT) best[u] = umax64(best[u], key);
    }
  }
#pragma unroll
  for (int u = 0; u < MT; ++u) {
    unsigned long long k = best[u];
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) k = umax64(k, __shfl_xor(k, d, 64));
    const int m = 16 * u + 4 * (cx.lane >> 4) + (cx.wave & 3);
    if ((cx.lane & 15) == 0 && m < a.M && k != 0ull) atomicMax(&s_best[m], k);
  }
  __syncthreads();
  greedy_publish_and_finish(a.out, s_best, 0, a.M, (unsigned)a.n_blocks, s_g);
}

struct GreedyArgs {
  const void* logits;
  const uint8_t* mask;
  int dtype;
  int M, V;
  int per_block;  // vocabulary entries per workgroup
  GreedyOut out;
};

constexpr int kGreedyPerBlock = 4096;

__global__ __launch_bounds__(kGreedyThreads) void greedy_kernel(GreedyArgs a) {
  __shared__ unsigned long long s_best[kMaxGreedyRows];
  const int m = blockIdx.y;
  const int v0 = blockIdx.x * a.per_block;
  const int v1 = min(a.V, v0 + a.per_block);
  const int tid = threadIdx.x;
  if (tid < kMaxGreedyRows) s_best[tid] = 0ull;
  __syncthreads();
  float neg;
  if (a.dtype == DFMI_BF16) neg = Num<BF16>::h2f(Num<BF16>::f2h(-1e9f));
  else if (a.dtype == DFMI_F16) neg = Num<F16>::h2f(Num<F16>::f2h(-1e9f));
  else neg = -1e9f;
  unsigned long long best = 0ull;
  const int64_t row = (int64_t)m * a.V;
  for (int v = v0 + tid; v < v1; v += kGreedyThreads) {
    float x;
    if (a.dtype == DFMI_BF16) x = Num<BF16>::h2f(static_cast<const uint16_t*>(a.logits)[row + v]);
    else if (a.dtype == DFMI_F16) x = Num<F16>::h2f(static_cast<const uint16_t*>(a.logits)[row + v]);
    else x = static_cast<const float*>(a.logits)[row + v];
    if (a.mask && a.mask[v]) x = neg;
    best = umax64(best, argmax_key(x, (uint32_t)v));
  }
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) best = umax64(best, __shfl_xor(best, d, 64));
  if ((tid & 63) == 0) atomicMax(&s_best[m], best);
  __syncthreads();
  __shared__ GreedyLds s_g;
  greedy_publish_and_finish(a.out, s_best, m, m + 1, gridDim.x * gridDim.y, &s_g);
}

__global__ void accept_kernel(const uint32_t* drafted, const uint32_t* posterior, int64_t L,
                              int32_t* out) {
  if (threadIdx.x == 0 && blockIdx.x == 0) {
    int64_t a = 0;
    while (a < L && drafted[a] == posterior[a]) ++a;
    out[0] = (int32_t)a;
  }
}

static size_t greedy_ws(int64_t M) { return 256 + round_up((size_t)M * 8u, 256); }

static int bind_out(GreedyOut& o, void* ws, size_t ws_bytes, int64_t M, uint32_t* posterior,
                    int32_t* accept_len, uint32_t* bonus, const uint32_t* verify_ids) {
  if (!ws || ws_bytes < greedy_ws(M) || (reinterpret_cast<uintptr_t>(ws) & 7u)) {
    set_error("greedy: workspace of %zu bytes (8-byte aligned) required, got %zu",
              greedy_ws(M), ws_bytes);
    return DFMI_ENOSPC;
  }
  o.counter = static_cast<uint32_t*>(ws);
  o.keys = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + 256);
  o.posterior = posterior;
  o.accept_len = accept_len;
  o.bonus = bonus;
  o.verify_ids = verify_ids;
  o.M = (int)M;
  return DFMI_OK;
}

template <typename Tag, int GS, int MT>
static void launch_lm(bool kfull, int blocks, int waves, hipStream_t st, const LmArgs& a) {
  if (kfull)
    hipLaunchKernelGGL((lmhead_greedy_kernel<Tag, GS, MT, true>), dim3(blocks), dim3(64 * waves),
                       0, st, a);
  else
    hipLaunchKernelGGL((lmhead_greedy_kernel<Tag, GS, MT, false>), dim3(blocks), dim3(64 * waves),
                       0, st, a);
}

template <typename Tag>
static void launch_lm_tag(int gs, int mt, bool kfull, int blocks, int waves, hipStream_t st,
                          const LmArgs& a) {
  if (gs == 32) {
    if (mt == 1) launch_lm<Tag, 32, 1>(kfull, blocks, waves, st, a);
    else launch_lm<Tag, 32, 2>(kfull, blocks, waves, st, a);
  } else if (gs == 64) {
    if (mt == 1) launch_lm<Tag, 64, 1>(kfull, blocks, waves, st, a);
    else launch_lm<Tag, 64, 2>(kfull, blocks, waves, st, a);
  } else {
    if (mt == 1) launch_lm<Tag, 128, 1>(kfull, blocks, waves, st, a);
    else launch_lm<Tag, 128, 2>(kfull, blocks, waves, st, a);
  }
}

template <typename Tag, int GS, int MT, int WV, bool TSB = false, int RW = 1>
static void launch_lm_stream_t(int blocks, hipStream_t st, const LmArgs& a) {
  constexpr int lds = Stream<Tag, GS, MT, WV, kSbPieces, 4, RW, TSB>::LDS_BYTES;
  // dynamic LDS above 64 KiB needs the kernel attribute raised (once)
  static const hipError_t attr = hipFuncSetAttribute(
      reinterpret_cast<const void*>(&lmhead_stream_kernel<Tag, GS, MT, WV, TSB, RW>),
      hipFuncAttributeMaxDynamicSharedMemorySize, lds);
  (void)attr;
  hipLaunchKernelGGL((lmhead_stream_kernel<Tag, GS, MT, WV, TSB, RW>), dim3(blocks),
                     dim3(64 * WV), lds, st, a.h, a.w, a.t, a.s, a.b, a.M, a.K, a.V, a.mask,
                     a.logits, a.softcap, a.chunks, a.n_blocks, a.out.keys, a.out.counter,
                     a.out.posterior, a.out.accept_len, a.out.bonus, a.out.verify_ids, a.out.M);
}

// With the pair table (gs 64 / 128, one activation block): 128-row blocks,
// 8 wavefronts in two row groups, two workgroups per CU.
template <typename Tag>
static void launch_lm_pairs(int gs, int blocks, hipStream_t st, const LmArgs& a) {
  if (gs == 64) launch_lm_stream_t<Tag, 64, 1, 8, true, 2>(blocks, st, a);
  else launch_lm_stream_t<Tag, 128, 1, 8, true, 2>(blocks, st, a);
}

// 4 wavefronts (two workgroups per CU): the vocabulary gives thousands of
// workgroups, so the whole K stays in one workgroup (no split epilogue).
template <typename Tag>
static void launch_lm_stream(int gs, int mt, int blocks, hipStream_t st, const LmArgs& a) {
  if (gs == 32) {
    if (mt == 1) launch_lm_stream_t<Tag, 32, 1, 4>(blocks, st, a);
    else launch_lm_stream_t<Tag, 32, 2, 4>(blocks, st, a);
  } else if (gs == 64) {
    if (mt == 1) launch_lm_stream_t<Tag, 64, 1, 4>(blocks, st, a);
    else launch_lm_stream_t<Tag, 64, 2, 4>(blocks, st, a);
  } else {
    if (mt == 1) launch_lm_stream_t<Tag, 128, 1, 4>(blocks, st, a);
    else launch_lm_stream_t<Tag, 128, 2, 4>(blocks, st, a);
  }
}

}  // namespace dfmi

using namespace dfmi;

extern "C" size_t dfmi_greedy_workspace_bytes(int64_t M) { return greedy_ws(M); }
extern "C" size_t dfmi_lmhead_workspace_bytes(int64_t M) { return greedy_ws(M); }

extern "C" int dfmi_greedy_accept(const void* logits, int logits_dtype, const uint8_t* suppress_mask,
                                  const uint32_t* verify_ids, int64_t M, int64_t V,
                                  uint32_t* posterior, int32_t* accept_len, uint32_t* bonus,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (logits_dtype != DFMI_BF16 && logits_dtype != DFMI_F16 && logits_dtype != DFMI_F32) {
    set_error("dfmi_greedy_accept: dtype %d unsupported", logits_dtype);
    return DFMI_EINVAL;
  }
  if (M < 1 || M > kMaxGreedyRows || V < 1 || V >= (1ll << 31) || M * V >= (1ll << 40)) {
    set_error("dfmi_greedy_accept: bad shape M=%lld V=%lld (1 <= M <= %d)", (long long)M,
              (long long)V, kMaxGreedyRows);
    return DFMI_EINVAL;
  }
  if (!logits || !posterior) {
    set_error("dfmi_greedy_accept: null pointer");
    return DFMI_EINVAL;
  }
  GreedyArgs a;
  int rc = bind_out(a.out, workspace, workspace_bytes, M, posterior, accept_len, bonus, verify_ids);
  if (rc != DFMI_OK) return rc;
  a.logits = logits;
  a.mask = suppress_mask;
  a.dtype = logits_dtype;
  a.M = (int)M;
  a.V = (int)V;
  a.per_block = kGreedyPerBlock;
  const dim3 grid((unsigned)((V + kGreedyPerBlock - 1) / kGreedyPerBlock), (unsigned)M);
  hipLaunchKernelGGL(greedy_kernel, grid, dim3(kGreedyThreads), 0, static_cast<hipStream_t>(stream),
                     a);
  return check_launch("dfmi_greedy_accept");
}

extern "C" int dfmi_lmhead_greedy_accept_pairs(
    const void* h, int h_dtype, const uint32_t* w_q, const void* scales, const void* biases,
    const uint32_t* sb_pairs, const uint8_t* suppress_mask, float softcap,
    const uint32_t* verify_ids, int64_t M, int64_t K, int64_t V, int group_size, int bits,
    uint32_t* posterior, int32_t* accept_len, uint32_t* bonus, void* logits_out, void* workspace,
    size_t workspace_bytes, void* stream) {
  if (h_dtype != DFMI_BF16 && h_dtype != DFMI_F16) {
    set_error("dfmi_lmhead_greedy_accept: dtype %d unsupported (bf16 or f16)", h_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4 || (group_size != 32 && group_size != 64 && group_size != 128)) {
    set_error("dfmi_lmhead_greedy_accept: bits=%d group_size=%d unsupported", bits, group_size);
    return DFMI_EINVAL;
  }
  if (M < 1 || M > kMaxGreedyRows || V < 1 || K < 32 || K % 32 || K % group_size ||
      V >= (1ll << 31) || K >= (1ll << 31) || V * (K / 8) > 0xFFFFFFFFll) {
    set_error("dfmi_lmhead_greedy_accept: bad shape M=%lld K=%lld V=%lld", (long long)M,
              (long long)K, (long long)V);
    return DFMI_EINVAL;
  }
  if (!h || !w_q || !scales || !biases || !posterior) {
    set_error("dfmi_lmhead_greedy_accept: null pointer");
    return DFMI_EINVAL;
  }
  if (!aligned16(h) || !aligned16(w_q) || !aligned16(scales) || !aligned16(biases) ||
      (sb_pairs && !aligned16(sb_pairs))) {
    set_error("dfmi_lmhead_greedy_accept: h, w_q, scales, biases and sb_pairs must be 16-byte "
              "aligned");
    return DFMI_EINVAL;
  }
  LmArgs a;
  int rc = bind_out(a.out, workspace, workspace_bytes, M, posterior, accept_len, bonus, verify_ids);
  if (rc != DFMI_OK) return rc;
  a.h = static_cast<const uint16_t*>(h);
  a.w = w_q;
  a.s = static_cast<const uint16_t*>(scales);
  a.b = static_cast<const uint16_t*>(biases);
  a.t = sb_pairs;
  a.mask = suppress_mask;
  a.logits = static_cast<uint16_t*>(logits_out);
  a.softcap = softcap;
  a.M = (int)M;
  a.K = (int)K;
  a.V = (int)V;
  a.chunks = (int)((K + kChunkK - 1) / kChunkK);
  const int nb_cols = 16 * kLmTiles;  // = kStreamRows
  a.n_blocks = (int)((V + nb_cols - 1) / nb_cols);
  const bool kfull = (K % kChunkK) == 0;
  const int mt = M <= 16 ? 1 : 2;
  hipStream_t st = static_cast<hipStream_t>(stream);
  // with the pair table: the pair-streaming loop, 128 vocabulary rows per
  // workgroup (the same logits, summed in the same order, as the window loop
  // below); only where that window loop takes the shape too (K / group_size
  // within one scale window), so that the logits never depend on whether a
  // table was given
  if (sb_pairs && M <= 16 && group_size >= 64 && stream_eligible(M, K, V, group_size) &&
      K / group_size <= sb_max_groups(kSbPieces)) {
    a.n_blocks = (int)((V + 2 * kStreamRows - 1) / (2 * kStreamRows));
    if (h_dtype == DFMI_BF16) launch_lm_pairs<BF16>(group_size, a.n_blocks, st, a);
    else launch_lm_pairs<F16>(group_size, a.n_blocks, st, a);
    return check_launch("dfmi_lmhead_greedy_accept");
  }
  // the streaming loop takes the whole K range in one scale / bias window
  if (stream_eligible(M, K, V, group_size) && K / group_size <= sb_max_groups(kSbPieces)) {
    if (h_dtype == DFMI_BF16) launch_lm_stream<BF16>(group_size, mt, a.n_blocks, st, a);
    else launch_lm_stream<F16>(group_size, mt, a.n_blocks, st, a);
    return check_launch("dfmi_lmhead_greedy_accept");
  }
  const int waves = a.chunks < kMaxWaves ? a.chunks : kMaxWaves;
  if (h_dtype == DFMI_BF16) launch_lm_tag<BF16>(group_size, mt, kfull, a.n_blocks, waves, st, a);
  else launch_lm_tag<F16>(group_size, mt, kfull, a.n_blocks, waves, st, a);
  return check_launch("dfmi_lmhead_greedy_accept");
}

extern "C" int dfmi_lmhead_greedy_accept(const void* h, int h_dtype, const uint32_t* w_q,
                                         const void* scales, const void* biases,
                                         const uint8_t* suppress_mask, float softcap,
                                         const uint32_t* verify_ids, int64_t M, int64_t K,
                                         int64_t V, int group_size, int bits, uint32_t* posterior,
                                         int32_t* accept_len, uint32_t* bonus, void* logits_out,
                                         void* workspace, size_t workspace_bytes, void* stream) {
  return dfmi_lmhead_greedy_accept_pairs(h, h_dtype, w_q, scales, biases, nullptr, suppress_mask,
                                         softcap, verify_ids, M, K, V, group_size, bits,
                                         posterior, accept_len, bonus, logits_out, workspace,
                                         workspace_bytes, stream);
}

extern "C" int dfmi_match_acceptance_length(const uint32_t* drafted, const uint32_t* posterior,
                                            int64_t L, int32_t* out, void* stream) {
  if (L < 0 || !out || (L > 0 && (!drafted || !posterior))) {
    set_error("dfmi_match_acceptance_length: bad arguments");
    return DFMI_EINVAL;
  }
  hipLaunchKernelGGL(accept_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream),
                     drafted, posterior, L, out);
  return check_launch("dfmi_match_acceptance_length");
}
