// The rest of the stock quantized matmul: the inputs the verify kernels do
// not take.  dflash-mlx hands anything its verify kernels decline to
// mx.quantized_matmul (dflash_mlx/verify_qmm.py:915-919, 936-938, 957-959,
// 984-986, 1005-1007), which also computes
//   * activations or scales in float32, or activations and scales of two
//     different 16-bit dtypes (MLX promotes both to the wider type: the
//     result is float32), and
//   * transpose = false: y = x . dequant(w) with w_q [K, N*bits/32] quantised
//     along its last axis (N), scales / biases [K, N/gs].
// Both run here in fp32 VALU arithmetic (these shapes are not on the verify
// path; every product the verify path makes goes through the MFMA kernels).
//
// transpose = true (qmm_t_general_kernel): a workgroup of 2 wavefronts owns
// 8 weight rows and 16 activation rows, the wavefronts taking alternate
// 256-k chunks; lane l takes row l / 8 and the 32-k piece l % 8 of a chunk,
// so the 8 lanes of a row read its 128 chunk bytes as one line.  Each
// wavefront stages its chunk of x in its own LDS as fp32 with each piece's
// sum; per piece and activation row the lane forms s * sum_k x q + b *
// sum_k x (the group's affine term split over its pieces).  At the end the
// second wavefront's sums are added to the first's and the 8 pieces of a row
// by a butterfly over its 8 lanes (every lane ends with the same bits).
//
// transpose = false (qmm_n_general_kernel): a workgroup of 16 wavefronts
// owns 8 words of every weight row (64 output columns at 4 bits, 32 at 8)
// and 4 activation rows; wavefront w takes the w-th sixteenth of K, lane l
// word l % 8 and every 8th k from l / 8 on, dequantises w[k][n] = q s + b
// per code (as the dequantised matrix MLX multiplies); the 8 k phases of a
// word are summed by a butterfly over their lanes and the 16 wavefronts in
// LDS in a fixed tree order.  Every result is deterministic.
#include <type_traits>

#include "dfmi_device.h"
#include "dfmi_host.h"

namespace dfmi {

struct F32 {};

// Storage of a float dtype and its conversions.
template <typename T> struct Elem;
template <> struct Elem<BF16> {
  using T = uint16_t;
  __device__ static inline float f(T v) { return __uint_as_float((uint32_t)v << 16); }
  __device__ static inline T of(float v) { return Num<BF16>::f2h(v); }
};
template <> struct Elem<F16> {
  using T = uint16_t;
  __device__ static inline float f(T v) { return (float)__builtin_bit_cast(_Float16, v); }
  __device__ static inline T of(float v) { return Num<F16>::f2h(v); }
};
template <> struct Elem<F32> {
  using T = float;
  __device__ static inline float f(T v) { return v; }
  __device__ static inline T of(float v) { return v; }
};

constexpr int kGtRows = 8;   // weight rows per workgroup (lane l: row l / 8)
constexpr int kGtWaves = 2;  // wavefronts of a workgroup, splitting the K chunks
constexpr int kGtM = 16;     // activation rows per workgroup
constexpr int kGtK = 256;    // k per staged chunk: 8 pieces of 32
constexpr int kGtPad = 36;   // floats per (row, piece) of the chunk: 32 + 4, pieces on distinct banks

template <typename X, typename S, typename Y, int BITS>
__global__ __launch_bounds__(64 * kGtWaves) void qmm_t_general_kernel(
    const typename Elem<X>::T* __restrict__ x, const uint32_t* __restrict__ w,
    const typename Elem<S>::T* __restrict__ sc, const typename Elem<S>::T* __restrict__ bi,
    typename Elem<Y>::T* __restrict__ y, int M, int K, int N, int gs) {
  // per wavefront: its staged chunk and the chunk's piece sums
  __shared__ float xs_all[kGtWaves][kGtM][8][kGtPad];
  __shared__ float xp_all[kGtWaves][kGtM][8];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row = lane >> 3, p = lane & 7;
  const int n = blockIdx.x * kGtRows + row;
  const int m0 = blockIdx.y * kGtM;
  const bool nok = n < N;
  const int64_t wpr = (int64_t)K * BITS / 32;  // words per weight row
  const int G = K / gs;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  float (*xs)[8][kGtPad] = xs_all[wave];
  float (*xp)[8] = xp_all[wave];
  float out[kGtM];
#pragma unroll
  for (int m = 0; m < kGtM; ++m) out[m] = 0.f;
  for (int k0 = wave * kGtK; k0 < K; k0 += kGtWaves * kGtK) {
    {  // stage x[m0 .. m0+15][k0 .. k0+255]: lane l takes row l / 4 and 64 consecutive k
      const int sm = lane >> 2, sk = (lane & 3) * 64;
      const int gm = m0 + sm;
#pragma unroll
      for (int h = 0; h < 4; ++h) {  // 16 k at a time
        const int gk = k0 + sk + 16 * h;
        float v[16];
        if (gm < M && gk < K) {  // K % 32 == 0: all 16 k inside
          const typename Elem<X>::T* src = x + (int64_t)gm * K + gk;
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = Elem<X>::f(src[j]);
        } else {
#pragma unroll
          for (int j = 0; j < 16; ++j) v[j] = 0.f;
        }
        const int kk = sk + 16 * h;
        float* dst = &xs[sm][kk >> 5][kk & 31];
#pragma unroll
        for (int j = 0; j < 16; ++j) dst[j] = v[j];
      }
    }
    // (the chunk is this wavefront's alone, and its LDS accesses complete in
    // order: no workgroup barrier)
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int h = 0; h < 2; ++h) {  // piece sums: lane l takes (row, piece) l and l + 64
      const int e = lane + 64 * h, sm = e >> 3, sp = e & 7;
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < 32; ++j) s += xs[sm][sp][j];
      xp[sm][sp] = s;
    }
    __builtin_amdgcn_wave_barrier();
    const int kk = k0 + 32 * p;
    if (nok && kk < K) {
      // the piece's 32 codes: 4 words (4-bit) or 8 (8-bit), 16-byte loads
      uint32_t wd[BITS];
      const uint4* src = reinterpret_cast<const uint4*>(w + (int64_t)n * wpr + kk * BITS / 32);
#pragma unroll
      for (int i = 0; i < BITS / 4; ++i) {
        const uint4 v = src[i];
        wd[4 * i] = v.x;
        wd[4 * i + 1] = v.y;
        wd[4 * i + 2] = v.z;
        wd[4 * i + 3] = v.w;
      }
      float q[32];
#pragma unroll
      for (int i = 0; i < 32; ++i) q[i] = (float)((wd[i * BITS / 32] >> ((i * BITS) % 32)) & kMask);
      const int64_t gi = (int64_t)n * G + kk / gs;
      const float s = Elem<S>::f(sc[gi]), b = Elem<S>::f(bi[gi]);
#pragma unroll
      for (int m = 0; m < kGtM; ++m) {
        const float* xr = xs[m][p];
        float a = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) a = fmaf(xr[i], q[i], a);
        out[m] = fmaf(s, a, fmaf(b, xp[m][p], out[m]));
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // wavefront 1's sums onto wavefront 0's (fixed order), then the row's 8
  // pieces by a butterfly over its 8 lanes (commutative adds: every lane
  // holds the same sum)
  __syncthreads();
  float* red = &xs_all[0][0][0][0];  // [kGtM][64]
  if (wave == 1) {
#pragma unroll
    for (int m = 0; m < kGtM; ++m) red[m * 64 + lane] = out[m];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int m = 0; m < kGtM; ++m) {
    float v = out[m] + red[m * 64 + lane];
    v += __shfl_xor(v, 1);
    v += __shfl_xor(v, 2);
    v += __shfl_xor(v, 4);
    out[m] = v;
  }
  if (nok) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int m = p + 8 * h;
      if (m0 + m < M) y[(int64_t)(m0 + m) * N + n] = Elem<Y>::of(out[m]);
    }
  }
}

constexpr int kGnM = 4;       // activation rows per workgroup
constexpr int kGnWaves = 16;  // wavefronts splitting K
constexpr int kGnWords = 8;   // words of a weight row per workgroup (lane l: word l % 8)
constexpr int kGnPh = 8;      // lanes per word, interleaved along k (lane l: k phase l / 8)
constexpr int kGnK = 64;      // k a wavefront stages at a time (8 per lane)

template <typename X, typename S, typename Y, int BITS>
__global__ __launch_bounds__(64 * kGnWaves) void qmm_n_general_kernel(
    const typename Elem<X>::T* __restrict__ x, const uint32_t* __restrict__ w,
    const typename Elem<S>::T* __restrict__ sc, const typename Elem<S>::T* __restrict__ bi,
    typename Elem<Y>::T* __restrict__ y, int M, int K, int N, int gs) {
  constexpr int VPW = 32 / BITS;  // codes per word
  constexpr int PER = kGnK / kGnPh;  // k per lane and staged chunk
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  // per wavefront: x[m0 .. m0+3][k] of its staged k (kGnK float4);
  // afterwards the tree reduction's partial sums (8 x 8 lanes x 4 x VPW)
  __shared__ float4 lds[kGnWaves * kGnK];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int jl = lane % kGnWords, ph = lane / kGnWords;
  const int64_t nw = (int64_t)N / VPW;  // words per row of w_q
  const int j = blockIdx.x * kGnWords + jl;
  const bool jok = j < nw;
  const int NG = N / gs;
  const int g = j * VPW / gs;  // the word's VPW columns share one group (VPW <= gs)
  const int m0 = blockIdx.y * kGnM;
  const int kper = (K + kGnWaves - 1) / kGnWaves;
  const int kb0 = wave * kper, kend = min(K, kb0 + kper);
  float acc[kGnM][VPW];
#pragma unroll
  for (int m = 0; m < kGnM; ++m)
#pragma unroll
    for (int v = 0; v < VPW; ++v) acc[m][v] = 0.f;
  float4* xs = lds + wave * kGnK;
  for (int kb = kb0; kb < kend; kb += kGnK) {
    {  // lane l stages x[m0 .. m0+3][kb + l]
      const int k = kb + lane;
      float v[kGnM];
#pragma unroll
      for (int m = 0; m < kGnM; ++m)
        v[m] = (k < kend && m0 + m < M) ? Elem<X>::f(x[(int64_t)(m0 + m) * K + k]) : 0.f;
      xs[lane] = make_float4(v[0], v[1], v[2], v[3]);
    }
    // (only this wavefront reads its slot; its LDS accesses complete in order)
    __builtin_amdgcn_wave_barrier();
    uint32_t wv[PER];
    float sv[PER], bv[PER];
#pragma unroll
    for (int u = 0; u < PER; ++u) {  // the lane's loads of the chunk first: k = kb + ph + 8 u
      const int k = kb + ph + kGnPh * u;
      const bool ok = jok && k < kend;
      wv[u] = ok ? w[(int64_t)k * nw + j] : 0u;
      sv[u] = ok ? Elem<S>::f(sc[(int64_t)k * NG + g]) : 0.f;
      bv[u] = ok ? Elem<S>::f(bi[(int64_t)k * NG + g]) : 0.f;
    }
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const float4 xv = xs[ph + kGnPh * u];  // (k past kend: staged 0, weight 0)
#pragma unroll
      for (int v = 0; v < VPW; ++v) {
        const float wq = fmaf((float)((wv[u] >> (v * BITS)) & kMask), sv[u], bv[u]);
        acc[0][v] = fmaf(xv.x, wq, acc[0][v]);
        acc[1][v] = fmaf(xv.y, wq, acc[1][v]);
        acc[2][v] = fmaf(xv.z, wq, acc[2][v]);
        acc[3][v] = fmaf(xv.w, wq, acc[3][v]);
      }
    }
    __builtin_amdgcn_wave_barrier();
  }
  // the 8 k phases of a word: a butterfly over lanes jl + 8 ph (commutative
  // adds: every phase ends with the same bits)
#pragma unroll
  for (int m = 0; m < kGnM; ++m)
#pragma unroll
    for (int v = 0; v < VPW; ++v) {
      float t = acc[m][v];
      t += __shfl_xor(t, 8);
      t += __shfl_xor(t, 16);
      t += __shfl_xor(t, 32);
      acc[m][v] = t;
    }
  // then the 16 wavefronts, a tree in LDS: w += w + h for h = 8, 4, 2, 1
  constexpr int VALS = kGnM * VPW;
  float* red = reinterpret_cast<float*>(lds);  // [8][kGnWords][VALS]
  for (int h = kGnWaves / 2; h >= 1; h >>= 1) {
    __syncthreads();
    if (wave >= h && wave < 2 * h && ph == 0) {
#pragma unroll
      for (int m = 0; m < kGnM; ++m)
#pragma unroll
        for (int v = 0; v < VPW; ++v)
          red[((wave - h) * kGnWords + jl) * VALS + m * VPW + v] = acc[m][v];
    }
    __syncthreads();
    if (wave < h && ph == 0) {
#pragma unroll
      for (int m = 0; m < kGnM; ++m)
#pragma unroll
        for (int v = 0; v < VPW; ++v)
          acc[m][v] += red[(wave * kGnWords + jl) * VALS + m * VPW + v];
    }
  }
  if (wave == 0 && ph == 0 && jok) {
#pragma unroll
    for (int m = 0; m < kGnM; ++m)
      if (m0 + m < M) {
#pragma unroll
        for (int v = 0; v < VPW; ++v)
          y[(int64_t)(m0 + m) * N + j * VPW + v] = Elem<Y>::of(acc[m][v]);
      }
  }
}

template <typename X, typename S, typename Y>
static void launch_general_t(bool transpose, int bits, const void* x, const uint32_t* w,
                             const void* s, const void* b, void* y, int M, int K, int N, int gs,
                             hipStream_t st) {
  using XT = typename Elem<X>::T;
  using ST = typename Elem<S>::T;
  using YT = typename Elem<Y>::T;
  const XT* xp = static_cast<const XT*>(x);
  const ST* sp = static_cast<const ST*>(s);
  const ST* bp = static_cast<const ST*>(b);
  YT* yp = static_cast<YT*>(y);
  if (transpose) {
    const dim3 grid((N + kGtRows - 1) / kGtRows, (M + kGtM - 1) / kGtM);
    if (bits == 8)
      hipLaunchKernelGGL((qmm_t_general_kernel<X, S, Y, 8>), grid, dim3(64 * kGtWaves), 0, st, xp,
                         w, sp, bp, yp, M, K, N, gs);
    else
      hipLaunchKernelGGL((qmm_t_general_kernel<X, S, Y, 4>), grid, dim3(64 * kGtWaves), 0, st, xp,
                         w, sp, bp, yp, M, K, N, gs);
  } else {
    const int nw = N / (32 / bits);
    const dim3 grid((nw + kGnWords - 1) / kGnWords, (M + kGnM - 1) / kGnM);
    if (bits == 8)
      hipLaunchKernelGGL((qmm_n_general_kernel<X, S, Y, 8>), grid, dim3(64 * kGnWaves), 0, st, xp,
                         w, sp, bp, yp, M, K, N, gs);
    else
      hipLaunchKernelGGL((qmm_n_general_kernel<X, S, Y, 4>), grid, dim3(64 * kGnWaves), 0, st, xp,
                         w, sp, bp, yp, M, K, N, gs);
  }
}

// y's dtype: the common dtype when x and the scales share one, else float32
template <typename X, typename S>
static void launch_general_s(bool transpose, int bits, const void* x, const uint32_t* w,
                             const void* s, const void* b, void* y, int M, int K, int N, int gs,
                             hipStream_t st) {
  if constexpr (std::is_same<X, S>::value)
    launch_general_t<X, S, X>(transpose, bits, x, w, s, b, y, M, K, N, gs, st);
  else
    launch_general_t<X, S, F32>(transpose, bits, x, w, s, b, y, M, K, N, gs, st);
}

template <typename X>
static void launch_general_x(int s_dtype, bool transpose, int bits, const void* x,
                             const uint32_t* w, const void* s, const void* b, void* y, int M,
                             int K, int N, int gs, hipStream_t st) {
  if (s_dtype == DFMI_BF16)
    launch_general_s<X, BF16>(transpose, bits, x, w, s, b, y, M, K, N, gs, st);
  else if (s_dtype == DFMI_F16)
    launch_general_s<X, F16>(transpose, bits, x, w, s, b, y, M, K, N, gs, st);
  else
    launch_general_s<X, F32>(transpose, bits, x, w, s, b, y, M, K, N, gs, st);
}

}  // namespace dfmi

using namespace dfmi;

extern "C" int dfmi_qmm_general(const void* x, int x_dtype, const uint32_t* w_q,
                                const void* scales, const void* biases, int s_dtype, void* y,
                                int64_t M, int64_t K, int64_t N, int group_size, int bits,
                                int transpose, void* workspace, size_t workspace_bytes,
                                void* stream) {
  auto dtype_ok = [](int d) { return d == DFMI_BF16 || d == DFMI_F16 || d == DFMI_F32; };
  if (!dtype_ok(x_dtype) || !dtype_ok(s_dtype)) {
    set_error("dfmi_qmm_general: dtypes x %d, scales %d unsupported (bf16, f16, f32)", x_dtype,
              s_dtype);
    return DFMI_EINVAL;
  }
  if (bits != 4 && bits != 8) {
    set_error("dfmi_qmm_general: bits=%d unsupported (4 or 8)", bits);
    return DFMI_EINVAL;
  }
  if (group_size != 32 && group_size != 64 && group_size != 128) {
    set_error("dfmi_qmm_general: group_size=%d unsupported (32, 64, 128)", group_size);
    return DFMI_EINVAL;
  }
  // the quantised axis: K (transpose) or N
  const int64_t Q = transpose ? K : N;
  if (M < 0 || N < 0 || K < 1 || Q % group_size || M >= (1ll << 31) || N >= (1ll << 31) ||
      K >= (1ll << 31) || N * K * bits / 32 >= (1ll << 40)) {
    set_error("dfmi_qmm_general: bad shape M=%lld K=%lld N=%lld gs=%d transpose=%d",
              (long long)M, (long long)K, (long long)N, group_size, transpose);
    return DFMI_EINVAL;
  }
  // the verify kernels' own case
  if (transpose && x_dtype == s_dtype && x_dtype != DFMI_F32)
    return dfmi_qmm_affine_ex(x, x_dtype, w_q, scales, biases, y, M, K, N, group_size, bits,
                              workspace, workspace_bytes, nullptr, stream);
  if (M == 0 || N == 0) return DFMI_OK;
  if ((M + kGnM - 1) / kGnM > 65535) {  // the grid's second dimension
    set_error("dfmi_qmm_general: M=%lld too large", (long long)M);
    return DFMI_EINVAL;
  }
  if (!x || !w_q || !scales || !biases || !y) {
    set_error("dfmi_qmm_general: null pointer");
    return DFMI_EINVAL;
  }
  if (transpose && !aligned16(w_q)) {  // 16-byte loads of 32-k pieces
    set_error("dfmi_qmm_general: w_q must be 16-byte aligned");
    return DFMI_EINVAL;
  }
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const bool tr = transpose != 0;
  const int m = (int)M, k = (int)K, n = (int)N;
  if (x_dtype == DFMI_BF16)
    launch_general_x<BF16>(s_dtype, tr, bits, x, w_q, scales, biases, y, m, k, n, group_size, st);
  else if (x_dtype == DFMI_F16)
    launch_general_x<F16>(s_dtype, tr, bits, x, w_q, scales, biases, y, m, k, n, group_size, st);
  else
    launch_general_x<F32>(s_dtype, tr, bits, x, w_q, scales, biases, y, m, k, n, group_size, st);
  return check_launch("dfmi_qmm_general");
}
