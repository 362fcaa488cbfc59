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


/*
 * Reverse-mode adjoint of the diagonal scan in float64, for full-size gradient checks -- the same
 * recurrences as brute.scan_bwd_brute (and as selective_scan_bwd_kernel.cuh:405-880 computes):
 *   g_t  = dout_t silu(z_t) (dout_t without z);  dz_t = dout_t y_t silu'(z_t)
 *   gh_t = C_t g_t + a_{t+1} gh_{t+1}, gh past the end = 0        (per state, a_t = exp(dt'_t A))
 *   dC_t += g_t h_t;  dB_t += gh_t dt'_t u_t;  du_t = D g_t + dt'_t sum_n gh_t B_t
 *   ddt'_t = sum_n gh_t (u_t B_t + A a_t h_{t-1});  dA += gh_t dt'_t a_t h_{t-1}
 *   ddelta_t = ddt'_t sigmoid(delta_t + bias) with softplus (1 past the threshold 20);
 *   dD += g_t u_t;  dbias += ddelta_t
 * The R rows must share one B and one C slice (row strides 0: the rows of one (batch, group));
 * dB and dC, (N, L) each, receive the sum over the R rows (added to what they hold). du, ddelta
 * and dz are (R, L), dA (R, N), dD and dbias (R,), each written for every row (dz only with z).
 */
void mm_oracle_scan_bwd_rows_f64(int64_t R, int64_t L, int64_t N,
                                 const double *u, const double *delta, const double *z,
                                 const double *A, const double *B, int64_t B_n_stride, int64_t B_l_stride,
                                 const double *C, int64_t C_n_stride, int64_t C_l_stride,
                                 const double *D, const double *bias, int softplus, const double *dout,
                                 double *du, double *ddelta, double *dz, double *dA, double *dD,
                                 double *dbias, double *dB, double *dC) {
#pragma omp parallel
    {
        double *accB = (double *)calloc((size_t)(N * L), sizeof(double));
        double *accC = (double *)calloc((size_t)(N * L), sizeof(double));
        double *H = (double *)malloc((size_t)(N * L) * sizeof(double));
        double *dts = (double *)malloc((size_t)L * sizeof(double));
        double *gs = (double *)malloc((size_t)L * sizeof(double));
        double *carry = (double *)malloc((size_t)N * sizeof(double));
#pragma omp for schedule(dynamic, 1)
        for (int64_t r = 0; r < R; ++r) {
            const double *ur = u + r * L, *dr = delta + r * L, *zr = z ? z + r * L : NULL, *gr = dout + r * L;
            const double *Ar = A + r * N;
            const double Dv = D ? D[r] : 0.0, bv = bias ? bias[r] : 0.0;
            for (int64_t n = 0; n < N; ++n) carry[n] = 0.0;
            /* forward: states at every step, gated output gradient g and dz */
            for (int64_t t = 0; t < L; ++t) {
                const double raw = dr[t] + bv;
                const double dt = softplus ? softplus64(raw) : raw;
                dts[t] = dt;
                double y = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const double prev = t > 0 ? H[(t - 1) * N + n] : 0.0;
                    const double h = exp(dt * Ar[n]) * prev + dt * ur[t] * B[n * B_n_stride + t * B_l_stride];
                    H[t * N + n] = h;
                    y += h * C[n * C_n_stride + t * C_l_stride];
                }
                y += Dv * ur[t];
                if (zr) {
                    const double sg = 1.0 / (1.0 + exp(-zr[t]));
                    gs[t] = gr[t] * zr[t] * sg;
                    if (dz) dz[r * L + t] = gr[t] * y * sg * (1.0 + zr[t] * (1.0 - sg));
                } else {
                    gs[t] = gr[t];
                }
            }
            /* reverse walk */
            double dAr[256] = {0.0}, dDr = 0.0, dbr = 0.0;
            for (int64_t t = L - 1; t >= 0; --t) {
                const double dt = dts[t], g = gs[t];
                double sgB = 0.0, ddt = 0.0;
                for (int64_t n = 0; n < N; ++n) {
                    const double Bn = B[n * B_n_stride + t * B_l_stride], Cn = C[n * C_n_stride + t * C_l_stride];
                    const double gh = Cn * g + carry[n];
                    const double a = exp(dt * Ar[n]);
                    const double prev = t > 0 ? H[(t - 1) * N + n] : 0.0;
                    accC[n * L + t] += g * H[t * N + n];
                    accB[n * L + t] += gh * dt * ur[t];
                    sgB += gh * Bn;
                    ddt += gh * (ur[t] * Bn + Ar[n] * a * prev);
                    dAr[n] += gh * dt * a * prev;
                    carry[n] = a * gh;
                }
                du[r * L + t] = Dv * g + dt * sgB;
                const double raw = dr[t] + bv;
                const double dd = softplus ? (raw > 20.0 ? ddt : ddt / (1.0 + exp(-raw))) : ddt;
                ddelta[r * L + t] = dd;
                dDr += g * ur[t];
                dbr += dd;
            }
            for (int64_t n = 0; n < N; ++n) dA[r * N + n] = dAr[n];
            if (dD) dD[r] = dDr;
            if (dbias) dbias[r] = dbr;
        }
#pragma omp critical
        {
            for (int64_t i = 0; i < N * L; ++i) {
                dB[i] += accB[i];
                dC[i] += accC[i];
            }
        }
        free(accB); free(accC); free(H); free(dts); free(gs); free(carry);
    }
}
