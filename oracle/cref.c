/*
 * Plain-C brute-force restatements used to pin the numpy oracle
 * (oracle/oracle.py) — TEST INFRASTRUCTURE ONLY, never linked into
 * libmbhip.so.  Loaded by tests/ through ctypes from oracle/lib/liboracle.so.
 *
 *   oracle_gemm_f64            C = A @ B, textbook triple loop
 *                              (reference mlx/kernels/common/sqr_mm.py:10-11)
 *   oracle_conv2d_nhwc_f64     direct 7-loop cross-correlation, NHWC x OHWI,
 *                              stride + zero padding
 *                              (reference mlx/kernels/common/conv2d.py:11-12)
 *   oracle_transpose_f32       B[j][i] = A[i][j], bitwise
 *                              (reference mlx/kernels/common/transpose_2d.py:10-11)
 */
#include <stddef.h>
#include <stdint.h>

void oracle_gemm_f64(const double* a, const double* b, double* c, int64_t m, int64_t n,
                     int64_t k) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t j = 0; j < n; ++j) {
            double acc = 0.0;
            for (int64_t p = 0; p < k; ++p) acc += a[i * k + p] * b[p * n + j];
            c[i * n + j] = acc;
        }
}

void oracle_conv2d_nhwc_f64(const double* x, const double* w, double* y, int64_t n, int64_t h,
                            int64_t wd, int64_t c, int64_t o, int64_t r, int64_t s,
                            int64_t stride, int64_t pad) {
    const int64_t p_out = (h + 2 * pad - r) / stride + 1;
    const int64_t q_out = (wd + 2 * pad - s) / stride + 1;
    for (int64_t b = 0; b < n; ++b)
        for (int64_t p = 0; p < p_out; ++p)
            for (int64_t q = 0; q < q_out; ++q)
                for (int64_t oc = 0; oc < o; ++oc) {
                    double acc = 0.0;
                    for (int64_t i = 0; i < r; ++i) {
                        const int64_t hi = p * stride + i - pad;
                        if (hi < 0 || hi >= h) continue;
                        for (int64_t j = 0; j < s; ++j) {
                            const int64_t wi = q * stride + j - pad;
                            if (wi < 0 || wi >= wd) continue;
                            const double* xr = x + ((b * h + hi) * wd + wi) * c;
                            const double* wr = w + ((oc * r + i) * s + j) * c;
                            for (int64_t ch = 0; ch < c; ++ch) acc += xr[ch] * wr[ch];
                        }
                    }
                    y[((b * p_out + p) * q_out + q) * o + oc] = acc;
                }
}

void oracle_transpose_f32(const float* a, float* b, int64_t rows, int64_t cols) {
    for (int64_t i = 0; i < rows; ++i)
        for (int64_t j = 0; j < cols; ++j) b[j * rows + i] = a[i * cols + j];
}
