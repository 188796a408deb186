/*
 * CPU restatement of the affine group-quantized matmul (TEST INFRASTRUCTURE /
 * CPU BASELINE ONLY -- never linked into the product library).
 *
 *   y[m, n] = sum_k x[m, k] * (q[n, k] * s[n, k / gs] + b[n, k / gs])
 *
 * Layout restated from dflash_mlx/verify_qmm.py:97-115 (4-bit) and 593-598
 * (8-bit): w_q uint32 [N, K*bits/32], first k in the lowest bits; scales and
 * biases [N, K/gs] in the activation dtype (bf16 here).  fp32 accumulation,
 * bf16 output rounded to nearest even -- the semantics of
 * mx.quantized_matmul on the MLX CPU stream that the reference falls back to
 * (verify_qmm.py:915-919).  OpenMP over output columns.
 *
 * The dot products keep LANES independent fp32 partial sums (lane l takes
 * k = l, l + LANES, ...) that are added in lane order at the end, so the
 * compiler vectorises the inner loop without reassociating anything, and a
 * dequantised weight row serves four activation rows per pass.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline float bf16_to_f32(uint16_t h) {
    uint32_t u = (uint32_t)h << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

#define LANES 16
#define MROWS 4

/* a[r] = sum_k x_r[k] w[k] for MROWS rows x_r = x + r * K (K % LANES == 0). */
static void dot_rows(const float *x, const float *w, int64_t K, int rows, float *a) {
    float part[MROWS][LANES];
    for (int r = 0; r < MROWS; ++r)
        for (int l = 0; l < LANES; ++l) part[r][l] = 0.0f;
    for (int64_t k = 0; k < K; k += LANES)
        for (int r = 0; r < MROWS; ++r) {
            if (r >= rows) break;
            const float *xr = x + r * K + k;
            for (int l = 0; l < LANES; ++l) part[r][l] += xr[l] * w[k + l];
        }
    for (int r = 0; r < rows; ++r) {
        float t = 0.0f;
        for (int l = 0; l < LANES; ++l) t += part[r][l];
        a[r] = t;
    }
}

static inline uint16_t f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* Returns 0 on success, -1 on an unsupported argument. */
int oracle_qmm_bf16(const uint16_t *x, const uint32_t *w_q, const uint16_t *scales,
                    const uint16_t *biases, uint16_t *y, int64_t M, int64_t K, int64_t N,
                    int group_size, int bits, int nthreads) {
    if (M <= 0 || K <= 0 || N <= 0) return 0;
    if (!(bits == 2 || bits == 4 || bits == 8)) return -1;
    if (group_size <= 0 || K % group_size != 0 || K % (32 / bits) != 0) return -1;
    const int64_t per = 32 / bits;
    const int64_t words = K / per;
    const int64_t groups = K / group_size;
    const uint32_t mask = (1u << bits) - 1u;

    float *xf = (float *)malloc(sizeof(float) * (size_t)(M * K));
    if (!xf) return -1;
    for (int64_t i = 0; i < M * K; ++i) xf[i] = bf16_to_f32(x[i]);

#ifdef _OPENMP
    if (nthreads > 0) omp_set_num_threads(nthreads);
#else
    (void)nthreads;
#endif
    int failed = 0;
#pragma omp parallel
    {
        float *wrow = (float *)malloc(sizeof(float) * (size_t)K);
        float *acc = (float *)malloc(sizeof(float) * (size_t)M);
        if (!wrow || !acc) {
#pragma omp atomic write
            failed = 1;
        } else {
#pragma omp for schedule(static)
            for (int64_t n = 0; n < N; ++n) {
                const uint32_t *wr = w_q + n * words;
                for (int64_t g = 0; g < groups; ++g) {
                    const float s = bf16_to_f32(scales[n * groups + g]);
                    const float b = bf16_to_f32(biases[n * groups + g]);
                    if (bits == 4 && group_size % 8 == 0) {
                        /* whole words: value i of word j at bits 4i */
                        const uint32_t *wg = wr + g * group_size / 8;
                        float *dst = wrow + g * group_size;
                        for (int64_t j = 0; j < group_size / 8; ++j)
                            for (int i = 0; i < 8; ++i)
                                dst[8 * j + i] = (float)((wg[j] >> (4 * i)) & 15u) * s + b;
                    } else {
                        for (int64_t k = g * group_size; k < (g + 1) * group_size; ++k) {
                            const uint32_t q = (wr[k / per] >> (bits * (k % per))) & mask;
                            wrow[k] = (float)q * s + b;
                        }
                    }
                }
                if (K % LANES == 0) {
                    for (int64_t m = 0; m < M; m += MROWS)
                        dot_rows(xf + m * K, wrow, K, (int)(M - m < MROWS ? M - m : MROWS),
                                 acc + m);
                } else {
                    for (int64_t m = 0; m < M; ++m) {
                        const float *xr = xf + m * K;
                        float a = 0.0f;
                        for (int64_t k = 0; k < K; ++k) a += xr[k] * wrow[k];
                        acc[m] = a;
                    }
                }
                for (int64_t m = 0; m < M; ++m) y[m * N + n] = f32_to_bf16(acc[m]);
            }
        }
        free(wrow);
        free(acc);
    }
    free(xf);
    return failed ? -1 : 0;
}

int oracle_max_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
