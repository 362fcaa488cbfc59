/*
 * scan_f64.c -- float64 sequential restatement of the selective scan, one (batch, dim) row at a
 * time -- TEST INFRASTRUCTURE ONLY (checker for sampled rows at the full benchmark shapes and
 * the "port" CPU baseline). Never linked into the product library.
 *
 * Follows selective_scan_ref, mamba_ssm/ops/selective_scan_interface.py:353-451 (real A, no P/Q):
 *   delta' = softplus(delta + bias)   (threshold 20, ssi.py:368-374)
 *   h_t[n] = exp(delta'_t A[n]) h_{t-1}[n] + delta'_t u_t B[n, t]    (ssi.py:388-396, 422-433)
 *   y_t    = sum_n h_t[n] C[n, t]                                    (ssi.py:435-440)
 *   out_t  = y_t + D u_t ;  outz_t = out_t * z_t / (1 + exp(-z_t))   (ssi.py:447-449)
 * The caller gathers each row's group slice of B/C (g(d) = d // (dim / G), ssi.py:395-400) and
 * passes element strides, so constant (dim, N) B/C use l_stride = 0.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

static double softplus64(double x) { return x > 20.0 ? x : log1p(exp(x)); }

void mm_oracle_scan_rows_f64(int64_t R, int64_t L, int64_t N,
                             const double *u, const double *delta, const double *z,
                             const double *A,
                             const double *B, int64_t B_row_stride, int64_t B_n_stride,
                             int64_t B_l_stride,
                             const double *C, int64_t C_row_stride, int64_t C_n_stride,
                             int64_t C_l_stride,
                             const double *D, const double *bias, int softplus,
                             double *out, double *outz, double *last,
                             int64_t chunk, double *hchunk) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < R; ++r) {
        double *h = (double *)calloc((size_t)N, sizeof(double));
        const double *ur = u + r * L;
        const double *dr = delta + r * L;
        const double *Ar = A + r * N;
        const double *Br = B + r * B_row_stride;
        const double *Cr = C + r * C_row_stride;
        const int64_t n_chunks = chunk > 0 ? (L + chunk - 1) / chunk : 0;
        for (int64_t t = 0; t < L; ++t) {
            double dt = dr[t] + (bias ? bias[r] : 0.0);
            if (softplus) dt = softplus64(dt);
            const double du = dt * ur[t];
            double y = 0.0;
            for (int64_t n = 0; n < N; ++n) {
                h[n] = exp(dt * Ar[n]) * h[n] + du * Br[n * B_n_stride + t * B_l_stride];
                y += h[n] * Cr[n * C_n_stride + t * C_l_stride];
            }
            if (D) y += D[r] * ur[t];
            out[r * L + t] = y;
            if (z && outz) {
                const double zz = z[r * L + t];
                outz[r * L + t] = y * zz / (1.0 + exp(-zz));
            }
            if (hchunk && chunk > 0 && (t == L - 1 || (t + 1) % chunk == 0)) {
                const int64_t c = t / chunk;
                for (int64_t n = 0; n < N; ++n) hchunk[(r * n_chunks + c) * N + n] = h[n];
            }
        }
        if (last)
            for (int64_t n = 0; n < N; ++n) last[r * N + n] = h[n];
        free(h);
    }
}

/*
 * Low-rank coupled (MotifMamba P/Q) variant, following selective_scan_full_matrix_cuda,
 * mamba_ssm/ops/selective_scan_interface.py:262-350:
 *   h_t = exp(delta'_t A) * h_{t-1} + delta'_t W h_{t-1} + delta'_t u_t B_t     (ssi.py:320-337)
 * with W = P Q formed once per row as a dense N x N matrix (the reference applies Q then P to the
 * state; the product is the same linear map). P is (N, K) and Q (K, N) per row (row strides
 * P_row_stride / Q_row_stride, 0 for a shared pair). hchunk receives h at each chunk end.
 */
void mm_oracle_scan_pq_rows_f64(int64_t R, int64_t L, int64_t N, int64_t K,
                                const double *u, const double *delta, const double *z,
                                const double *A,
                                const double *B, int64_t B_row_stride, int64_t B_n_stride,
                                int64_t B_l_stride,
                                const double *C, int64_t C_row_stride, int64_t C_n_stride,
                                int64_t C_l_stride,
                                const double *P, int64_t P_row_stride,
                                const double *Q, int64_t Q_row_stride,
                                const double *D, const double *bias, int softplus,
                                double *out, double *outz, double *last,
                                int64_t chunk, double *hchunk) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int64_t r = 0; r < R; ++r) {
        double *h = (double *)calloc((size_t)N, sizeof(double));
        double *hn = (double *)calloc((size_t)N, sizeof(double));
        double *W = (double *)calloc((size_t)(N * N), sizeof(double));
        const double *Pr = P + r * P_row_stride;
        const double *Qr = Q + r * Q_row_stride;
        for (int64_t i = 0; i < N; ++i)
            for (int64_t j = 0; j < N; ++j) {
                double acc = 0.0;
                for (int64_t k = 0; k < K; ++k) acc += Pr[i * K + k] * Qr[k * N + j];
                W[i * N + j] = acc;
            }
        const double *ur = u + r * L;
        const double *dr = delta + r * L;
        const double *Ar = A + r * N;
        const double *Br = B + r * B_row_stride;
        const double *Cr = C + r * C_row_stride;
        const int64_t n_chunks = chunk > 0 ? (L + chunk - 1) / chunk : 0;
        for (int64_t t = 0; t < L; ++t) {
            double dt = dr[t] + (bias ? bias[r] : 0.0);
            if (softplus) dt = softplus64(dt);
            const double du = dt * ur[t];
            double y = 0.0;
            for (int64_t i = 0; i < N; ++i) {
                double wh = 0.0;
                for (int64_t j = 0; j < N; ++j) wh += W[i * N + j] * h[j];
                hn[i] = exp(dt * Ar[i]) * h[i] + dt * wh + du * Br[i * B_n_stride + t * B_l_stride];
            }
            for (int64_t i = 0; i < N; ++i) {
                h[i] = hn[i];
                y += h[i] * Cr[i * C_n_stride + t * C_l_stride];
            }
            if (D) y += D[r] * ur[t];
            out[r * L + t] = y;
            if (z && outz) {
                const double zz = z[r * L + t];
                outz[r * L + t] = y * zz / (1.0 + exp(-zz));
            }
            if (hchunk && chunk > 0 && (t == L - 1 || (t + 1) % chunk == 0)) {
                const int64_t c = t / chunk;
                for (int64_t n = 0; n < N; ++n) hchunk[(r * n_chunks + c) * N + n] = h[n];
            }
        }
        if (last)
            for (int64_t n = 0; n < N; ++n) last[r * N + n] = h[n];
        free(h);
        free(hn);
        free(W);
    }
}
